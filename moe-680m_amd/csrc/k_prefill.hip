// k_prefill.hip -- prefill path (M > 8): grouped IQ4_XS-dequant f16 MFMA GEMMs.
//
// Replaces the reference's bucketed prefill dispatches (src/inference.rs:683-732): per
// non-empty bucket a tiled w1_w3_fused GEMM into an f16 scratch and a w2_scatter GEMM
// whose epilogue read-modify-writes the f16 hidden state (shaders/w1_w3_fused.comp,
// shaders/w2_scatter.comp).  Here, after the bucket fill has produced expert-sorted slots
// and a list of tiles (up to PF_BM slots of one expert):
//   prep:    per token, x (RMSNorm fused when asked) times a power of two s_t that puts
//            max|x| in [2^14, 2^15), stored as f16 with K permuted inside 32-blocks (the
//            order the weight nibbles arrive in, see below); 1/s_t kept per token;
//   gate_up: per (tile, 128 gate/up column pairs) a workgroup of 8 waves; the tile's token
//            rows (gathered -- the reference's kernel skipped this gather) are staged in
//            LDS 128 K at a time, double-buffered, and shared by the 8 waves; every wave
//            decodes its own 16 W1 rows and 16 W3 rows straight into MFMA B fragments in
//            registers (no LDS, no barrier for weights) and runs v_mfma_f32_16x16x32_f16;
//            epilogue: silu(g) * u with the 1/s_t undone, f32 h, plus the per-row max|h|
//            of each 128-column block;
//   down:    per (tile, 256 output rows) the same over K = inter; the f32 h rows are
//            scaled per row by a power of two (from the row max) into f16 as they are
//            staged; epilogue multiplies by 2^-s_row * c * slot weight, one f32 row per slot;
//   combine: y_t (+)= sum over t's 9 slots in slot order -- deterministic, no atomics, no
//            f16 read-modify-write race (the reference's w2_scatter.comp:77-86 RMW).
//
// Operand precision: the weight dl*kv (exact in f32, up to 23 significant bits) is rounded
// once to f16 (dl itself is rounded to f16 first: <= 2^-10 relative in all); activations
// and h are f16 after an exact power-of-two scaling, so only their 11-bit rounding remains.
// MFMA accumulates in f32.
//
// Weight decode into a B fragment.  v_mfma_f32_16x16x32_f16 takes from lane (g, n) of the
// B operand 8 K values of column n; the K order inside one 32-wide MFMA step is free as long
// as A uses the same one.  Lane group g takes qs bytes 4g..4g+3 of the sub-block: low
// nibbles are K = 4g..4g+3, high nibbles K = 16+4g..16+4g+3, so one 32-bit qs load gives
// the lane its 8 weights.  The activations are stored in that order (perm32 below).
// Codebook bytes come from the v_perm lookup (kv + 128, see moe_device.hpp); a second
// v_perm places each byte under an 0x64 high byte, which is the f16 1024 + byte, exactly;
// one packed f16 add of -1152 gives kv exactly and one packed multiply applies dl.
#include "moe_internal.hpp"

namespace moe {

constexpr int PF_KC = 128;             // K per LDS stage
constexpr int PF_LDSK = PF_KC + 8;     // +16 B per row: 16 rows at one column hit 16 bank groups
constexpr int PF_WAVES = 8;
constexpr int PF_NGU = 16 * PF_WAVES;  // gate/up columns per workgroup
constexpr int PF_ND = 32 * PF_WAVES;   // down output rows per workgroup (2 N-tiles per wave)

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Position, in the stored order, of natural K index k inside a 32-block (and its inverse).
__host__ __device__ constexpr int perm32_pos(int k) {
    return (k & 16) ? 8 * ((k & 15) >> 2) + 4 + (k & 3) : 8 * (k >> 2) + (k & 3);
}

__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
    f16x2 v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

// 8 weights of one qs dword (low nibbles then high nibbles) as 4 packed f16 pairs, * dl.
__device__ __forceinline__ u32x4 dq8_f16(uint32_t q, uint32_t dl2) {
    uint32_t lo, hi;
    kv_biased8(q, lo, hi);
    constexpr uint32_t MAGIC = 0x64646464u;
    const f16x2 bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const f16x2 dl = __builtin_bit_cast(f16x2, dl2);
    const uint32_t p[4] = {__builtin_amdgcn_perm(MAGIC, lo, 0x04010400u), __builtin_amdgcn_perm(MAGIC, lo, 0x04030402u),
                           __builtin_amdgcn_perm(MAGIC, hi, 0x04010400u), __builtin_amdgcn_perm(MAGIC, hi, 0x04030402u)};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const f16x2 v = (__builtin_bit_cast(f16x2, p[i]) + bias) * dl;
        o[i] = __builtin_bit_cast(uint32_t, v);
    }
    return u32x4{o[0], o[1], o[2], o[3]};
}

// dl = d * (ls - 32) of sub-block j from an 8-byte header, rounded once to f16, in both
// halves of the returned word.
__device__ __forceinline__ uint32_t dl_pair(u32x2 hdr, int j) {
    const float dl = sub_scale(hdr, j);
    const uint32_t h = __builtin_bit_cast(uint16_t, (_Float16)dl);
    return h | (h << 16);
}

__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b),
                                                  c, 0, 0, 0);
}

// Power of two s with max * s in [2^14, 2^15) (1 when max is 0 or not finite); returns s,
// *inv = 1/s.  Exponents are clamped so both stay normal floats.
__device__ __forceinline__ float pow2_scale(float mx, float *inv) {
    int e = 0;
    if (!(mx > 0.0f) || !(mx < INFINITY)) {
        *inv = 1.0f;
        return 1.0f;
    }
    (void)frexpf(mx, &e); // mx = f * 2^e, f in [0.5, 1)
    int sh = 15 - e;
    sh = sh > 120 ? 120 : (sh < -120 ? -120 : sh);
    *inv = ldexpf(1.0f, -sh);
    return ldexpf(1.0f, sh);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float max16(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    return v;
}

// ---------------------------------------------------------------- prep
// One wave per token; lane owns 32-blocks lane, lane+64, ... of the row.
template <int H>
__global__ __launch_bounds__(256) void k_pf_prep(PrefillArgs a) {
    constexpr int NB = H / 32 / 64 > 0 ? H / 32 / 64 : 1; // 32-blocks per lane
    static_assert(H % (32 * 64) == 0 || H == 512, "prep shape");
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= a.M) return;
    constexpr int NBK = H / 32;
    float v[NB][32];
    const bool own = lane < NBK;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        if (own) load32(a.x + (size_t)t * H + 32 * (lane + 64 * b), v[b]);
        else
#pragma unroll
            for (int i = 0; i < 32; ++i) v[b][i] = 0.0f;
    }
    if (a.rmsnorm) {
        float ss = 0.f;
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int i = 0; i < 32; ++i) ss = __builtin_fmaf(v[b][i], v[b][i], ss);
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss * (1.0f / (float)H) + 1e-6f);
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int i = 0; i < 32; ++i) v[b][i] *= inv;
    }
    float mx = 0.f;
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < 32; ++i) mx = fmaxf(mx, fabsf(v[b][i]));
    mx = __builtin_bit_cast(float, wave_max_u32(__builtin_bit_cast(uint32_t, mx))); // non-negative: int order
    float inv_s;
    const float s = pow2_scale(mx, &inv_s);
    if (own) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            u32x4 o[4];
#pragma unroll
            for (int p = 0; p < 16; ++p) {
                // stored position 2p, 2p+1 <- natural k with perm32_pos(k) == 2p, 2p+1
                const int g = (2 * p) >> 3, j = (2 * p) & 7;
                const int k0 = j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4);
                o[p >> 2][p & 3] = pack_f16x2(v[b][k0] * s, v[b][k0 + 1] * s);
            }
            u32x4 *dst = reinterpret_cast<u32x4 *>(a.xh + (size_t)t * H + 32 * (lane + 64 * b));
#pragma unroll
            for (int i = 0; i < 4; ++i) dst[i] = o[i];
        }
    }
    if (lane == 0) a.xinv[t] = inv_s;
}

// ---------------------------------------------------------------- shared pipeline pieces
// Raw IQ4_XS data of one K stage (PF_KC = 128 K = 4 sub-blocks, half a super-block) for NR
// 16-row weight groups, read from the R16 layout (k_repack_r16): lane (g, n) gets the
// header of row n and, in one 16-byte load, dword g of each of the stage's 4 sub-blocks of
// row n -- exactly its B-fragment bytes for 4 MFMA K-steps.  A wave's load is 1 KB of
// contiguous memory.  Stages live in a ring of 4 so each is requested three stages ahead.
constexpr int R16_BLOCK = 16 * SB_BYTES; // one super-block column of a 16-row group

template <int NR>
struct WStage {
    u32x2 hdr[NR];
    u32x4 q[NR];
};

// groups[r]: first byte of the 16-row group (= matrix base + first row * row bytes).
template <int NR>
__device__ __forceinline__ void wstage_load(WStage<NR> &s, const uint8_t *const (&groups)[NR], int ch, int lane) {
    const int sb = ch >> 1, h = ch & 1;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const uint8_t *blk = groups[r] + (size_t)sb * R16_BLOCK;
        s.hdr[r] = ldg<u32x2>(blk + 8 * (lane & 15));
        s.q[r] = ldg<u32x4>(blk + 128 + 1024 * h + 16 * lane);
    }
}

// dl pairs of the stage's 4 sub-blocks: lane group g computes sub-block kb0 + g and every
// lane fetches the one of K-step ks from lane ks*16 + n.
template <int NR>
__device__ __forceinline__ void wstage_dl(const WStage<NR> &s, int ch, int g, int n, uint32_t (&dl)[NR][4]) {
    const int kb0 = (ch & 1) * 4;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const uint32_t mine = dl_pair(s.hdr[r], kb0 + g);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) dl[r][ks] = (uint32_t)__builtin_amdgcn_ds_bpermute((ks * 16 + n) * 4, (int)mine);
    }
}

// One stage of MFMAs: NR B fragments (dequantized here) against the MT M-tiles of the LDS
// A stage.  Each K-step first issues the A fragment reads, then the decode VALU work (which
// covers the LDS latency), then the MFMAs.
template <int NR, int MT, int LK>
__device__ __forceinline__ void stage_mfma(const WStage<NR> &s0, const uint32_t (&dl)[NR][4], const _Float16 *As,
                                           int n, int g, f32x4 (&acc)[MT][NR]) {
    uint32_t qv[NR][4];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        qv[r][0] = s0.q[r][0];
        qv[r][1] = s0.q[r][1];
        qv[r][2] = s0.q[r][2];
        qv[r][3] = s0.q[r][3];
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const _Float16 *ap = As + n * LK + 32 * ks + 8 * g;
        u32x4 av[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) av[mt] = *reinterpret_cast<const u32x4 *>(ap + 16 * mt * LK);
        u32x4 b[NR];
#pragma unroll
        for (int r = 0; r < NR; ++r) b[r] = dq8_f16(qv[r][ks], dl[r][ks]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < NR; ++r) acc[mt][r] = mfma16(av[mt], b[r], acc[mt][r]);
    }
}

// The K loop shared by both GEMMs, fully unrolled: with a rolled loop the compiler's vmcnt
// bookkeeping merges at the loop head and waits for every prefetch in flight.  Per stage ch: request the A rows of stage ch+2 (into
// register set ch&1) and the weights of stage ch+3 (ring slot (ch+3)&3), run the MFMAs of
// stage ch from LDS buffer ch&1, then move A of stage ch+1 into the other LDS buffer.  Loads
// are issued in the order they are needed, so a wave's in-order vmcnt waits never hold a
// use behind a later prefetch.  Only LDS traffic crosses the barriers.
template <int NCH, int NR, int MT, int LK, typename ALoad, typename AStore>
__device__ __forceinline__ void gemm_k_loop(const uint8_t *const (&rows)[NR], _Float16 (*As)[PF_BM * PF_LDSK], int n,
                                            int g, f32x4 (&acc)[MT][NR], ALoad aload, AStore astore) {
    WStage<NR> ws[4];
#pragma unroll
    for (int c = 0; c < 3; ++c)
        if (c < NCH) wstage_load(ws[c], rows, c, n + 16 * g);
    aload(std::integral_constant<int, 0>{}, 0);
    if (NCH > 1) aload(std::integral_constant<int, 1>{}, 1);
    astore(std::integral_constant<int, 0>{}, 0);
    lds_barrier();
    auto stage = [&](auto Sc, int ch) __attribute__((always_inline)) {
        constexpr int S = decltype(Sc)::value; // ch & 3
        if (ch + 2 < NCH) aload(std::integral_constant<int, S & 1>{}, ch + 2);
        __builtin_amdgcn_sched_barrier(0);
        uint32_t dl[NR][4];
        wstage_dl(ws[S], ch, g, n, dl);
        stage_mfma<NR, MT, LK>(ws[S], dl, As[S & 1], n, g, acc);
        __builtin_amdgcn_sched_barrier(0);
        if (ch + 3 < NCH) wstage_load(ws[(S + 3) & 3], rows, ch + 3, n + 16 * g);
        __builtin_amdgcn_sched_barrier(0);
        if (ch + 1 < NCH) astore(std::integral_constant<int, (S + 1) & 1>{}, (S + 1) & 1);
        lds_barrier();
    };
#pragma unroll
    for (int c0 = 0; c0 < NCH; c0 += 4) {
        stage(std::integral_constant<int, 0>{}, c0);
        if (c0 + 1 < NCH) stage(std::integral_constant<int, 1>{}, c0 + 1);
        if (c0 + 2 < NCH) stage(std::integral_constant<int, 2>{}, c0 + 2);
        if (c0 + 3 < NCH) stage(std::integral_constant<int, 3>{}, c0 + 3);
    }
}

// Big tiles hold PF_SMALL_MAX+1 .. PF_BM slots; the GEMM bodies are instantiated for 4 and 8
// M-tiles of 16 rows so that each inner loop is straight-line code (no per-M-tile branches).
template <typename F>
__device__ __forceinline__ void by_mtiles(int nrows, F f) {
    if (nrows <= 64) f(std::integral_constant<int, 4>{});
    else f(std::integral_constant<int, 8>{});
}

// ---------------------------------------------------------------- gate/up
template <int H, int I>
__global__ __launch_bounds__(64 * PF_WAVES, 1) void k_pf_gate_up(PrefillArgs a) {
    constexpr int MG = PF_BM;
    constexpr int KC = PF_KC, LK = PF_LDSK, NCH = H / KC;
    constexpr int ROWB = (H / QK) * SB_BYTES;
    static_assert(H % QK == 0 && I % PF_NGU == 0 && KC * 2 == QK, "gate/up shape");
    __shared__ __attribute__((aligned(16))) _Float16 As[2][MG * LK];
    __shared__ uint32_t rowmax[MG];

    const Tile tl = a.tiles[blockIdx.y];
    if (tl.expert < 0) return;
    const int e = tl.expert, row0 = tl.row0, nrows = tl.nrows;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int c0 = blockIdx.x * PF_NGU + wv * 16; // this wave's h columns
    if (tid < MG) rowmax[tid] = 0u;

    // A staging: thread -> (row ar, 32 K at column 32*ap of the stage)
    const int ar = tid >> 2, ap = tid & 3;
    const int aslot = row0 + (ar < nrows ? ar : nrows - 1);
    const _Float16 *asrc = a.xh + (size_t)a.sorted_tok[aslot] * H + 32 * ap;
    // Weights: rows c0 + n of W1 (gate) and W3 (up).
    const uint8_t *rows[2] = {expert_w(a.L.w1, a.L.s1, a.L.sw1, e, a.E) + (size_t)c0 * ROWB,
                              expert_w(a.L.w3, a.L.s3, a.L.sw3, e, a.E) + (size_t)c0 * ROWB};

    by_mtiles(nrows, [&](auto MTc) __attribute__((always_inline)) {
        constexpr int MT = decltype(MTc)::value;
        const bool arow = ar < 16 * MT; // only the rows of the M-tiles in use are moved
        u32x4 ra[2][4];
        auto aload = [&](auto Rc, int ch) __attribute__((always_inline)) {
            constexpr int R = decltype(Rc)::value;
            if (arow) {
                const u32x4 *p = reinterpret_cast<const u32x4 *>(asrc + ch * KC);
#pragma unroll
                for (int i = 0; i < 4; ++i) ra[R][i] = ldg<u32x4>(p + i);
            }
        };
        auto astore = [&](auto Rc, int buf) __attribute__((always_inline)) {
            constexpr int R = decltype(Rc)::value;
            if (arow) {
                u32x4 *d = reinterpret_cast<u32x4 *>(&As[buf][ar * LK + 32 * ap]);
#pragma unroll
                for (int i = 0; i < 4; ++i) d[i] = ra[R][i];
            }
        };
        f32x4 acc[MT][2];
#pragma unroll
        for (int i = 0; i < MT; ++i) acc[i][0] = acc[i][1] = f32x4{0, 0, 0, 0};
        gemm_k_loop<NCH, 2, MT, LK>(rows, As, n, g, acc, aload, astore);

        // epilogue: h = silu(g) * u with the token scale undone; per-row max|h| of the block
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = 16 * mt + 4 * g + i;
                float hv = 0.0f;
                if (m < nrows) {
                    const int slot = row0 + m;
                    const float inv = a.xinv[a.sorted_tok[slot]];
                    hv = silu(acc[mt][0][i] * inv) * (acc[mt][1][i] * inv);
                    a.hf[(size_t)slot * I + c0 + n] = hv;
                }
                const float rm = max16(fabsf(hv));
                if (n == 0) atomicMax(&rowmax[m], __builtin_bit_cast(uint32_t, rm));
            }
    });
    __syncthreads();
    if (tid < nrows) a.hmax[(size_t)(row0 + tid) * (I / PF_NGU) + blockIdx.x] = __builtin_bit_cast(float, rowmax[tid]);
}

// ---------------------------------------------------------------- down
template <int H, int I>
__global__ __launch_bounds__(64 * PF_WAVES, 1) void k_pf_down(PrefillArgs a) {
    constexpr int MG = PF_BM, NTW = 2;
    constexpr int KC = PF_KC, LK = PF_LDSK, NCH = I / KC;
    constexpr int ROWB = (I / QK) * SB_BYTES;
    constexpr int NHB = I / PF_NGU; // h max blocks per row
    static_assert(I % QK == 0 && H % PF_ND == 0 && KC * 2 == QK, "down shape");
    __shared__ __attribute__((aligned(16))) _Float16 As[2][MG * LK];
    __shared__ float s_scale[MG], s_inv[MG];

    const Tile tl = a.tiles[blockIdx.y];
    if (tl.expert < 0) return;
    const int e = tl.expert, row0 = tl.row0, nrows = tl.nrows;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int r0 = blockIdx.x * PF_ND + wv * 32; // this wave's output rows r0 .. r0+31

    if (tid < MG) {
        float mx = 0.f;
        if (tid < nrows)
#pragma unroll
            for (int b = 0; b < NHB; ++b) mx = fmaxf(mx, a.hmax[(size_t)(row0 + tid) * NHB + b]);
        float inv;
        s_scale[tid] = pow2_scale(mx, &inv);
        s_inv[tid] = inv;
    }
    __syncthreads();

    const int ar = tid >> 2, ap = tid & 3;
    const int aslot = row0 + (ar < nrows ? ar : nrows - 1);
    const float *asrc = a.hf + (size_t)aslot * I + 32 * ap;
    const float asc = s_scale[ar];
    const uint8_t *w2 = expert_w(a.L.w2, a.L.s2, a.L.sw2, e, a.E);
    const uint8_t *rows[NTW] = {w2 + (size_t)r0 * ROWB, w2 + (size_t)(r0 + 16) * ROWB};

    by_mtiles(nrows, [&](auto MTc) __attribute__((always_inline)) {
        constexpr int MT = decltype(MTc)::value;
        const bool arow = ar < 16 * MT;
        f32x4 ra[2][8];
        auto aload = [&](auto Rc, int ch) __attribute__((always_inline)) {
            constexpr int R = decltype(Rc)::value;
            if (arow) {
                const f32x4 *p = reinterpret_cast<const f32x4 *>(asrc + ch * KC);
#pragma unroll
                for (int i = 0; i < 8; ++i) ra[R][i] = ldg<f32x4>(p + i);
            }
        };
        auto astore = [&](auto Rc, int buf) __attribute__((always_inline)) {
            constexpr int R = decltype(Rc)::value;
            if (arow) {
                float v[32];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    v[4 * i + 0] = ra[R][i][0] * asc;
                    v[4 * i + 1] = ra[R][i][1] * asc;
                    v[4 * i + 2] = ra[R][i][2] * asc;
                    v[4 * i + 3] = ra[R][i][3] * asc;
                }
                u32x4 o[4];
#pragma unroll
                for (int p = 0; p < 16; ++p) {
                    const int gg = (2 * p) >> 3, j = (2 * p) & 7;
                    const int k0 = j < 4 ? 4 * gg + j : 16 + 4 * gg + (j - 4);
                    o[p >> 2][p & 3] = pack_f16x2(v[k0], v[k0 + 1]);
                }
                u32x4 *d = reinterpret_cast<u32x4 *>(&As[buf][ar * LK + 32 * ap]);
#pragma unroll
                for (int i = 0; i < 4; ++i) d[i] = o[i];
            }
        };
        f32x4 acc[MT][NTW];
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int t = 0; t < NTW; ++t) acc[i][t] = f32x4{0, 0, 0, 0};
        gemm_k_loop<NCH, NTW, MT, LK>(rows, As, n, g, acc, aload, astore);

#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = 16 * mt + 4 * g + i;
                if (m < nrows) {
                    const int slot = row0 + m;
                    const float sc = a.c * a.sorted_w[slot] * s_inv[m];
                    float *prow = a.part + (size_t)slot * H + r0 + n;
#pragma unroll
                    for (int t = 0; t < NTW; ++t) prow[16 * t] = sc * acc[mt][t][i];
                }
            }
    });
}

// ---------------------------------------------------------------- small tiles
// Tiles of at most PF_SM (16) slots: the tile's whole A operand (16 rows x K, f16) is staged in
// LDS once, after which the 8 waves run their K loops independently -- no barrier inside the
// loop, each wave only waits for its own weight loads, and two workgroups share a CU so one
// hides the other's load latency.
template <int NCH, int NR>
__device__ __forceinline__ void wring_prologue(WStage<NR> (&ws)[4], const uint8_t *const (&rows)[NR], int lane) {
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        if (c < NCH) wstage_load(ws[c], rows, c, lane);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// K loop over an LDS-resident A; the ring's first three stages were requested by
// wring_prologue (before the A staging, so both latencies overlap).
template <int NCH, int NR, int LK>
__device__ __forceinline__ void gemm_k_loop_resident(WStage<NR> (&ws)[4], const uint8_t *const (&rows)[NR],
                                                     const _Float16 *As, int n, int g, f32x4 (&acc)[1][NR]) {
    auto stage = [&](auto Sc, int ch) __attribute__((always_inline)) {
        constexpr int S = decltype(Sc)::value;
        uint32_t dl[NR][4];
        wstage_dl(ws[S], ch, g, n, dl);
        stage_mfma<NR, 1, LK>(ws[S], dl, As + ch * PF_KC, n, g, acc);
        // keep the scheduler from moving loads across stages: each stage's weights are
        // requested exactly three stages ahead, in the order they are consumed
        __builtin_amdgcn_sched_barrier(0);
        if (ch + 3 < NCH) wstage_load(ws[(S + 3) & 3], rows, ch + 3, n + 16 * g);
        __builtin_amdgcn_sched_barrier(0);
    };
#pragma unroll
    for (int c0 = 0; c0 < NCH; c0 += 4) {
        stage(std::integral_constant<int, 0>{}, c0);
        if (c0 + 1 < NCH) stage(std::integral_constant<int, 1>{}, c0 + 1);
        if (c0 + 2 < NCH) stage(std::integral_constant<int, 2>{}, c0 + 2);
        if (c0 + 3 < NCH) stage(std::integral_constant<int, 3>{}, c0 + 3);
    }
}

template <int H, int I>
__global__ __launch_bounds__(64 * PF_WAVES, 2) void k_pf_gate_up_s(PrefillArgs a) {
    constexpr int LKS = H + 8, NCH = H / PF_KC;
    constexpr int ROWB = (H / QK) * SB_BYTES;
    constexpr int CH = H / 32; // halves per staging thread (32 threads per row)
    static_assert(CH % 8 == 0, "small gate/up staging");
    __shared__ __attribute__((aligned(16))) _Float16 As[PF_SM * LKS];
    __shared__ uint32_t rowmax[PF_SM];

    const Tile tl = a.tiles[a.tile_max + blockIdx.y];
    if (tl.expert < 0) return;
    const int e = tl.expert, row0 = tl.row0, nrows = tl.nrows;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int c0 = blockIdx.x * PF_NGU + wv * 16;
    if (tid < PF_SM) rowmax[tid] = 0u;
    const uint8_t *rows[2] = {expert_w(a.L.w1, a.L.s1, a.L.sw1, e, a.E) + (size_t)c0 * ROWB,
                              expert_w(a.L.w3, a.L.s3, a.L.sw3, e, a.E) + (size_t)c0 * ROWB};
    WStage<2> ws[4];
    wring_prologue<NCH>(ws, rows, lane);
    {
        const int ar = tid >> 5, ac = (tid & 31) * CH;
        const int slot = row0 + (ar < nrows ? ar : nrows - 1);
        const u32x4 *src = reinterpret_cast<const u32x4 *>(a.xh + (size_t)a.sorted_tok[slot] * H + ac);
        u32x4 *dst = reinterpret_cast<u32x4 *>(As + ar * LKS + ac);
#pragma unroll
        for (int i = 0; i < CH / 8; ++i) dst[i] = ldg<u32x4>(src + i);
    }
    lds_barrier();
    f32x4 acc[1][2];
    acc[0][0] = acc[0][1] = f32x4{0, 0, 0, 0};
    gemm_k_loop_resident<NCH, 2, LKS>(ws, rows, As, n, g, acc);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = 4 * g + i;
        float hv = 0.0f;
        if (m < nrows) {
            const int slot = row0 + m;
            const float inv = a.xinv[a.sorted_tok[slot]];
            hv = silu(acc[0][0][i] * inv) * (acc[0][1][i] * inv);
            a.hf[(size_t)slot * I + c0 + n] = hv;
        }
        const float rm = max16(fabsf(hv));
        if (n == 0) atomicMax(&rowmax[m], __builtin_bit_cast(uint32_t, rm));
    }
    __syncthreads();
    if (tid < nrows) a.hmax[(size_t)(row0 + tid) * (I / PF_NGU) + blockIdx.x] = __builtin_bit_cast(float, rowmax[tid]);
}

template <int H, int I>
__global__ __launch_bounds__(64 * PF_WAVES, 2) void k_pf_down_s(PrefillArgs a) {
    constexpr int LKS = I + 8, NCH = I / PF_KC, NTW = 2;
    constexpr int ROWB = (I / QK) * SB_BYTES;
    constexpr int NHB = I / PF_NGU;
    constexpr int TPR = I / 32; // staging threads per row, one 32-block each
    __shared__ __attribute__((aligned(16))) _Float16 As[PF_SM * LKS];

    const Tile tl = a.tiles[a.tile_max + blockIdx.y];
    if (tl.expert < 0) return;
    const int e = tl.expert, row0 = tl.row0, nrows = tl.nrows;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int r0 = blockIdx.x * PF_ND + wv * 32;
    const uint8_t *w2 = expert_w(a.L.w2, a.L.s2, a.L.sw2, e, a.E);
    const uint8_t *rows[NTW] = {w2 + (size_t)r0 * ROWB, w2 + (size_t)(r0 + 16) * ROWB};
    WStage<NTW> ws[4];
    wring_prologue<NCH>(ws, rows, lane);
    if (tid < PF_SM * TPR) {
        const int ar = tid / TPR, ab = tid % TPR;
        const int slot = row0 + (ar < nrows ? ar : nrows - 1);
        float mx = 0.f;
#pragma unroll
        for (int b = 0; b < NHB; ++b) mx = fmaxf(mx, a.hmax[(size_t)slot * NHB + b]);
        float inv;
        const float sc = pow2_scale(mx, &inv);
        float v[32];
        load32(a.hf + (size_t)slot * I + 32 * ab, v);
        u32x4 o[4];
#pragma unroll
        for (int p = 0; p < 16; ++p) {
            const int gg = (2 * p) >> 3, j = (2 * p) & 7;
            const int k0 = j < 4 ? 4 * gg + j : 16 + 4 * gg + (j - 4);
            o[p >> 2][p & 3] = pack_f16x2(v[k0] * sc, v[k0 + 1] * sc);
        }
        u32x4 *d = reinterpret_cast<u32x4 *>(As + ar * LKS + 32 * ab);
#pragma unroll
        for (int i = 0; i < 4; ++i) d[i] = o[i];
    }
    lds_barrier();
    f32x4 acc[1][NTW];
    acc[0][0] = acc[0][1] = f32x4{0, 0, 0, 0};
    gemm_k_loop_resident<NCH, NTW, LKS>(ws, rows, As, n, g, acc);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = 4 * g + i;
        if (m < nrows) {
            const int slot = row0 + m;
            float mx = 0.f;
#pragma unroll
            for (int b = 0; b < NHB; ++b) mx = fmaxf(mx, a.hmax[(size_t)slot * NHB + b]);
            float inv;
            (void)pow2_scale(mx, &inv);
            const float sc = a.c * a.sorted_w[slot] * inv;
            float *prow = a.part + (size_t)slot * H + r0 + n;
#pragma unroll
            for (int t = 0; t < NTW; ++t) prow[16 * t] = sc * acc[0][t][i];
        }
    }
}

// ---------------------------------------------------------------- combine
// y_t (+)= sum_{s=0..8} part[pos[t][s]]; restates the weighted sum that the reference's
// w2_scatter epilogue accumulates into the hidden state (shaders/w2_scatter.comp:77-86),
// in a fixed order.
template <int H>
__global__ __launch_bounds__(256) void k_pf_combine(PrefillArgs a) {
    const int t = blockIdx.x;
    uint32_t ps[SLOTS];
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) ps[s] = a.pos[(size_t)t * SLOTS + s];
    for (int n4 = threadIdx.x; n4 < H / 4; n4 += 256) {
        f32x4 acc = f32x4{0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < SLOTS; ++s)
            if (ps[s] != 0xFFFFFFFFu) acc += ldg<f32x4>(a.part + (size_t)ps[s] * H + 4 * n4);
        f32x4 *yp = reinterpret_cast<f32x4 *>(a.y + (size_t)t * H) + n4;
        f32x4 base = a.accumulate ? *yp : f32x4{0, 0, 0, 0};
        *yp = base + acc;
    }
}

template <int H, int I>
static hipError_t launch_prefill_t(const PrefillArgs &a, hipStream_t st, hipStream_t aux, hipEvent_t ev_fork,
                                   hipEvent_t ev_join, KernelTimer *T) {
    {
        TimedLaunch tl(T, MOE_K_PREFILL_PREP, st);
        hipLaunchKernelGGL((k_pf_prep<H>), dim3((a.M + 3) / 4), dim3(256), 0, st, a);
    }
    // small tiles on the second stream, concurrently with the big tiles
    hipError_t he = hipEventRecord(ev_fork, st);
    if (he == hipSuccess) he = hipStreamWaitEvent(aux, ev_fork, 0);
    if (he != hipSuccess) return he;
    {
        TimedLaunch tl(T, MOE_K_PREFILL_GATE_UP_SMALL, aux);
        hipLaunchKernelGGL((k_pf_gate_up_s<H, I>), dim3(I / PF_NGU, a.stile_max), dim3(64 * PF_WAVES), 0, aux, a);
    }
    {
        TimedLaunch tl(T, MOE_K_PREFILL_DOWN_SMALL, aux);
        hipLaunchKernelGGL((k_pf_down_s<H, I>), dim3(H / PF_ND, a.stile_max), dim3(64 * PF_WAVES), 0, aux, a);
    }
    {
        TimedLaunch tl(T, MOE_K_PREFILL_GATE_UP, st);
        hipLaunchKernelGGL((k_pf_gate_up<H, I>), dim3(I / PF_NGU, a.tile_max), dim3(64 * PF_WAVES), 0, st, a);
    }
    {
        TimedLaunch tl(T, MOE_K_PREFILL_DOWN, st);
        hipLaunchKernelGGL((k_pf_down<H, I>), dim3(H / PF_ND, a.tile_max), dim3(64 * PF_WAVES), 0, st, a);
    }
    he = hipEventRecord(ev_join, aux);
    if (he == hipSuccess) he = hipStreamWaitEvent(st, ev_join, 0);
    if (he != hipSuccess) return he;
    {
        TimedLaunch tl(T, MOE_K_PREFILL_COMBINE, st);
        hipLaunchKernelGGL((k_pf_combine<H>), dim3(a.M), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

hipError_t launch_prefill(int H, int I, const PrefillArgs &a, hipStream_t st, hipStream_t aux, hipEvent_t ev_fork,
                          hipEvent_t ev_join, KernelTimer *T) {
    if (H == 2048 && I == 512) return launch_prefill_t<2048, 512>(a, st, aux, ev_fork, ev_join, T);
    if (H == 512 && I == 256) return launch_prefill_t<512, 256>(a, st, aux, ev_fork, ev_join, T);
    return hipErrorInvalidValue;
}

} // namespace moe
