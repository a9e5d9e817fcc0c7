// k_prefill.hip -- prefill path (M > 8): grouped IQ4_XS-dequant f16 MFMA GEMMs.
//
// Replaces the reference's bucketed prefill dispatches (src/inference.rs:683-732): per
// non-empty bucket a tiled w1_w3_fused GEMM into an f16 scratch and a w2_scatter GEMM
// whose epilogue read-modify-writes the f16 hidden state (shaders/w1_w3_fused.comp,
// shaders/w2_scatter.comp).  Here, after the chain's bucket fill (k_pf_count, k_pf_place,
// below) has produced expert-sorted slots and a list of tiles (up to PF_BM slots of one
// expert):
//   prep:    per token, x (RMSNorm fused when asked) times a power of two s_t that puts
//            max|x| in [2^14, 2^15), stored as f16 with K permuted inside 32-blocks (the
//            order the weight nibbles arrive in, see below); 1/s_t kept per token -- run in
//            the same launch as the slot placement (k_pf_place), which does not need it;
//   gate_up: per (tile, 64 gate/up column pairs; 128 when M > 768) a workgroup of 8 waves,
//            two per CU; the tile's token rows (gathered -- the reference's kernel skipped
//            this gather) are resident in LDS one 64 KB chunk of K at a time and shared by the
//            8 waves; each wave decodes 16 W1 rows and 16 W3 rows (with 64 columns, two waves
//            share them and take alternate 128-K stages; their sums meet in LDS) straight
//            into MFMA B fragments in registers (no LDS, no barrier for weights) and runs
//            v_mfma_f32_16x16x32_f16; epilogue: silu(g) * u with the 1/s_t undone, the
//            per-row max|h| of the item's column block, and h as f16 scaled by that max's
//            power of two, stored in the down kernel's K order;
//   down:    per (tile, 256 output rows) the same over K = inter (one chunk); each column
//            block of the f16 h rows is rescaled to the power of two of the row's max (a
//            factor 2^-j, exact for normal f16) as it is staged; epilogue multiplies by
//            2^-s_row * c * slot weight and writes each slot row as f16, every 32 columns
//            scaled by the power of two of their max (the exponent kept in a byte);
//   combine: y_t (+)= sum over t's 9 slots in slot order, in f32 -- deterministic, no
//            atomics, no f16 read-modify-write race (the reference's w2_scatter.comp:77-86).
//
// Operand precision: the weight dl*kv (exact in f32, up to 23 significant bits) is rounded
// once to f16 (dl itself is rounded to f16 first: <= 2^-10 relative in all), after an exact
// power-of-two shift 2^-s_n per weight row (row_shift below, undone in the epilogue);
// activations and h are f16 after an exact power-of-two scaling, so only their 11-bit
// rounding remains.  MFMA accumulates in f32.
//
// Weight decode into a B fragment.  v_mfma_f32_16x16x32_f16 takes from lane (g, n) of the
// B operand 8 K values of column n; the K order inside one 32-wide MFMA step is free as long
// as A uses the same one.  A lane takes one qs dword d of a sub-block: low nibbles are
// K = 4d..4d+3, high nibbles K = 16+4d..16+4d+3 of that sub-block, so one 32-bit qs word
// gives the lane its 8 weights (which sub-block and dword each lane group takes in each
// step: wstage_load).  The activations are stored in that order (perm32 below).
// Codebook bytes b = kv + 128 come from the v_perm lookup (moe_device.hpp); a second v_perm
// places each byte under a zero high byte, which is the f16 subnormal b * 2^-24, exactly; one
// packed f16 FMA  b * 2^-24 * B + C  with B = dl * 2^(24 - s_n) and C = -128 * 2^-24 * B (both
// exact f16) gives dl * kv * 2^-s_n with one rounding.  The row shift s_n (from the row's
// largest |d|) keeps B <= 65504, so no scale overflows, and the row's large weights normal.
#include "moe_internal.hpp"
#include "bucket_fill.hpp"

namespace moe {

constexpr int PF_KC = 128;             // K per LDS stage
constexpr int PF_WAVES = 8;
constexpr int PF_ND = 32 * PF_WAVES;   // down output rows per workgroup (2 N-tiles per wave)

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Position, in the stored order, of natural K index k inside a 32-block (and its inverse).
__host__ __device__ constexpr int perm32_pos(int k) {
    return (k & 16) ? 8 * ((k & 15) >> 2) + 4 + (k & 3) : 8 * (k >> 2) + (k & 3);
}

__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
    f16x2 v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

// 8 weights of one qs dword (low nibbles then high nibbles) as 4 packed f16 pairs
// dl * kv * 2^-s (b2, c2: the sub-block's B and C pairs, bc_pair).  v_perm selector 0x0c is a
// zero byte.
__device__ __forceinline__ u32x4 dq8_f16(uint32_t q, uint32_t b2, uint32_t c2) {
    uint32_t lo, hi;
    kv_biased8(q, lo, hi);
    const f16x2 bv = __builtin_bit_cast(f16x2, b2), cv = __builtin_bit_cast(f16x2, c2);
    const uint32_t p[4] = {__builtin_amdgcn_perm(lo, lo, 0x0c010c00u), __builtin_amdgcn_perm(lo, lo, 0x0c030c02u),
                           __builtin_amdgcn_perm(hi, hi, 0x0c010c00u), __builtin_amdgcn_perm(hi, hi, 0x0c030c02u)};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        o[i] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(f16x2, p[i]), bv, cv));
    return u32x4{o[0], o[1], o[2], o[3]};
}

// B = dl * F (F = 2^(24 - s), row_shift) of sub-block j from an 8-byte header, rounded once to
// f16 (dl = d * (ls - 32) is exact in f32 and F a power of two, so B = f16(dl) * F wherever
// both are normal), and C = -2^-17 * B = -128 * 2^-24 * B; each in both halves of a word.  C
// is exact down to |B| = 8, and below that off by at most 2^-25, against weights of the row
// up to 2^-1.
__device__ __forceinline__ void bc_pair(u32x2 hdr, int j, float F, uint32_t &b2, uint32_t &c2) {
    const _Float16 b = (_Float16)(sub_scale(hdr, j) * F);
    const f16x2 bv = {b, b};
    const f16x2 k = {(_Float16)-0x1p-17f, (_Float16)-0x1p-17f};
    b2 = __builtin_bit_cast(uint32_t, bv);
    c2 = __builtin_bit_cast(uint32_t, bv * k);
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

// The exponent of pow2_scale: max * 2^sh in [2^14, 2^15) (0 when max is 0 or not finite),
// sh in [-120, 120].
__device__ __forceinline__ int pow2_shift(float mx) {
    if (!(mx > 0.0f) || !(mx < INFINITY)) return 0;
    int e = 0;
    (void)frexpf(mx, &e);
    const int sh = 15 - e;
    return sh > 120 ? 120 : (sh < -120 ? -120 : sh);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
// Max over the 16 lanes of a DPP row, for non-negative floats (ordered as their bit patterns,
// so each step is one v_max_u32 with a DPP source).
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
}
__device__ __forceinline__ float max16(float v) {
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    u = max(u, dpp_u<0xB1>(u));
    u = max(u, dpp_u<0x4E>(u));
    u = max(u, dpp_u<0x141>(u));
    u = max(u, dpp_u<0x140>(u));
    return __builtin_bit_cast(float, u);
}

// ---------------------------------------------------------------- prep
// One wave per token.  Lane l holds quads l, l + 64, ... (four consecutive elements each) of the
// row, so every load instruction reads 1 KB of consecutive bytes; a quad's f16 values go
// straight to their place in the 32-block's stored order (perm32_pos: quad j < 4 of the block
// to positions 8j..8j+3, quad j >= 4 to 8(j-4)+4..+7), one 8-byte store each.
template <int H>
__device__ __forceinline__ void prep_token(const PrefillArgs &a, int t, int lane) {
    constexpr int NQ = H / 4, QPL = NQ / 64; // quads of the row; per lane
    static_assert(NQ % 64 == 0, "whole waves of quads");
    f32x4 v[QPL];
#pragma unroll
    for (int u = 0; u < QPL; ++u) v[u] = ldg<f32x4>(a.x + (size_t)t * H + 4 * (lane + 64 * u));
    if (a.rmsnorm) {
        float ss = 0.f;
#pragma unroll
        for (int u = 0; u < QPL; ++u)
#pragma unroll
            for (int i = 0; i < 4; ++i) ss = __builtin_fmaf(v[u][i], v[u][i], ss);
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss * (1.0f / (float)H) + 1e-6f);
#pragma unroll
        for (int u = 0; u < QPL; ++u)
#pragma unroll
            for (int i = 0; i < 4; ++i) v[u][i] *= inv;
    }
    float mx = 0.f;
#pragma unroll
    for (int u = 0; u < QPL; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, fabsf(v[u][i]));
    mx = __builtin_bit_cast(float, wave_max_u32(__builtin_bit_cast(uint32_t, mx))); // non-negative: int order
    float inv_s;
    const float s = pow2_scale(mx, &inv_s);
    const int j = lane & 7, pos = j < 4 ? 8 * j : 8 * (j - 4) + 4; // the quad's place in its 32-block
#pragma unroll
    for (int u = 0; u < QPL; ++u) {
        const int q = lane + 64 * u;
        const u32x2 o = {pack_f16x2(v[u][0] * s, v[u][1] * s), pack_f16x2(v[u][2] * s, v[u][3] * s)};
        *reinterpret_cast<u32x2 *>(a.xh + (size_t)t * H + 32 * (q >> 3) + pos) = o;
    }
    if (lane == 0) a.xinv[t] = inv_s;
}

// ---------------------------------------------------------------- the chain's bucket fill
// Replaces router::build_expert_batches (src/router.rs:55-97) inside the prefill chain, where
// only the tiles, each slot's sorted position and the sorted tokens and weights are needed --
// and where a slot's place inside its bucket changes no result (every GEMM row, its scaling
// and its partial are computed from that row alone, and the combine sums a token's slots in
// slot order).  So the slots are ranked by an atomic counter per bucket rather than in token
// order (moe_bucket_fill, the drop-in for build_expert_batches, keeps the token order), and the
// fill takes two launches of many workgroups whatever M is:
//   k_pf_count: one wave per token routes it (with logits, as k_router_topk) or reads its ids,
//       applies the pair rule (an id above n_experts, or one its token named in an earlier slot,
//       is dropped and flagged) and ranks each kept slot in its bucket: inside the workgroup by
//       an LDS counter, then by one add per touched bucket to the bucket's global counter;
//   k_pf_place: every placing workgroup scans the E + 1 counts itself (ranges; workgroup 0 also
//       writes the tile lists) and places its share of the slots -- sorted token, weight and
//       position -- with the prep of PF_PREP_TOKENS tokens per workgroup in the others.
// The counters start at zero and k_pf_combine, the chain's last launch, zeroes them again.
// The shared expert's bucket has no counter: token t's shared row is row t of it.
constexpr int PF_COUNT_TOKENS = 8; // tokens per counting workgroup, one wave each (16: 6.3 against 5.1 us at M = 512; 4: 10.3 against 8.7 us at M = 4096)
constexpr uint32_t PF_SLOT_HOLE = 0xFFFFFFFEu; // slot 8 of a token with no kept shared slot

template <bool ROUTE>
__global__ __launch_bounds__(64 * PF_COUNT_TOKENS) void k_pf_count(PfCountArgs c) {
    // Routed experts: per-workgroup bucket counts in LDS first, then one global add per bucket
    // the workgroup touched.  The shared expert's bucket takes no count: every token has one
    // row in it, at rank t -- its kept shared slot, or (only when its ids name no valid shared
    // slot) a hole row of weight 0 that no token reads back.  An add per shared slot would
    // serialise M adds on one counter.
    __shared__ uint32_t hist[MOE_MAX_EXPERTS + 1], base[MOE_MAX_EXPERTS + 1];
    const int lane = threadIdx.x & 63, E1 = c.E + 1;
    for (int e = threadIdx.x; e < E1; e += 64 * PF_COUNT_TOKENS) hist[e] = 0u;
    __syncthreads();
    const int t = blockIdx.x * PF_COUNT_TOKENS + (int)(threadIdx.x >> 6);
    const bool tok = t < c.M; // whole waves
    int id = 0;
    if (tok) {
        if constexpr (ROUTE) {
            float wt;
            route_wave<4>(c.logits + (size_t)t * c.E, c.E, c.renorm, lane, id, wt);
            if (lane < SLOTS) {
                c.ids[(size_t)t * SLOTS + lane] = (uint16_t)id;
                c.w[(size_t)t * SLOTS + lane] = wt;
            }
        } else {
            id = lane < SLOTS ? (int)c.ids[(size_t)t * SLOTS + lane] : 0;
        }
    }
    // the pair rule for given ids; routed ids are E distinct indices and the shared id, so no
    // slot of theirs is dropped (ROUTE skips the check)
    const bool bad = !ROUTE && tok && lane < SLOTS && id > c.E;
    bool dup = false;
    if constexpr (!ROUTE) {
#pragma unroll
        for (int s = 0; s < SLOTS - 1; ++s) {
            const int o = __builtin_amdgcn_readlane(id, s);
            dup = dup || (tok && s < lane && lane < SLOTS && !bad && o == id);
        }
    }
    const bool keep = tok && lane < SLOTS && !bad && !dup;
    const uint64_t nb = __ballot(bad), nd = __ballot(dup), ns = __ballot(keep && id == c.E);
    if (lane == 0 && (nb | nd))
        set_flag(c.flags, (nb ? (uint32_t)MOE_DEVFLAG_BAD_ID : 0u) | (nd ? (uint32_t)MOE_DEVFLAG_DUP_ID : 0u));
    const bool routed = keep && id != c.E;
    uint32_t rank = routed ? atomicAdd(&hist[id], 1u) : 0u;
    __syncthreads();
    // counter copy blockIdx % 8 (the workgroup's XCD): a hot bucket's adds are spread over
    // eight addresses instead of queueing on one
    const uint32_t cp = blockIdx.x % PF_CNT_COPIES;
    for (int e = threadIdx.x; e < E1; e += 64 * PF_COUNT_TOKENS) {
        const uint32_t n = hist[e];
        base[e] = n ? __hip_atomic_fetch_add((MOE_GLOBAL uint32_t *)(c.cnt + cp * E1 + e), n, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT)
                    : 0u;
    }
    __syncthreads();
    if (tok && lane < SLOTS) {
        uint32_t info = 0xFFFFFFFFu;
        if (routed) info = ((uint32_t)id << PF_SLOT_RANK_BITS) | (cp << PF_SLOT_COPY_SHIFT) | (base[id] + rank);
        else if (keep) info = ((uint32_t)c.E << PF_SLOT_RANK_BITS) | (uint32_t)t; // the shared slot
        else if (lane == SLOTS - 1 && !ns) info = PF_SLOT_HOLE;
        c.slot[(size_t)t * SLOTS + lane] = info;
    }
}

// Slots per placing workgroup (one per thread) and tokens per prep workgroup (its first four
// waves; the others leave at once): both are bound by the CU's address unit -- scattered
// 2- and 4-byte stores, and per wave 64 cache lines touched by each of a token's 8 loads and 4
// stores -- so they are spread over many CUs (measured, M = 512: 9.1 us for the launch with
// 4096 slots and 16 tokens per workgroup).
constexpr int PF_PLACE_SLOTS = 512; // slots per placing workgroup (1024: 12.8 against 12.3 us at M = 4096)
constexpr int PF_PREP_TOKENS = 4; // tokens per prep workgroup, one wave each (16: 14.0 against 12.8 us at M = 4096)

template <int H>
__global__ __launch_bounds__(BF_THREADS) void k_pf_place(BucketArgs b, PfCountArgs c, PrefillArgs a) {
    const int nplace = (SLOTS * b.M + PF_PLACE_SLOTS - 1) / PF_PLACE_SLOTS;
    const int blk = (int)blockIdx.x, tid = (int)threadIdx.x;
    if (blk >= nplace) {
        const int wv = tid >> 6, t = (blk - nplace) * PF_PREP_TOKENS + wv;
        if (wv < PF_PREP_TOKENS && t < a.M) prep_token<H>(a, t, tid & 63); // whole waves
        return;
    }
    extern __shared__ uint32_t smem[];
    const int E1 = b.E1;
    const BucketScan S = bucket_scan_lds(smem, E1);
    // per bucket the copies' counts: their total, and each copy's start inside the bucket
    uint32_t *cb = smem + 5 * (E1 + 1); // [PF_CNT_COPIES][E1]
    for (int e = tid; e < E1; e += BF_THREADS) {
        uint32_t tot = 0u;
        if (e < E1 - 1)
#pragma unroll
            for (int k = 0; k < PF_CNT_COPIES; ++k) {
                cb[k * E1 + e] = tot;
                tot += ldg<uint32_t>(c.cnt + k * E1 + e);
            }
        S.tot[e] = e == E1 - 1 ? (uint32_t)b.M : tot;
    }
    __syncthreads();
    bucket_lists(b, S, blk == 0);
    const int n = SLOTS * b.M, i0 = blk * PF_PLACE_SLOTS, i1 = min(i0 + PF_PLACE_SLOTS, n);
    for (int i = i0 + tid; i < i1; i += BF_THREADS) {
        const uint32_t info = ldg<uint32_t>(c.slot + i);
        const float wv = ldg<float>(c.w + i);
        const int t = i / SLOTS;
        uint32_t p = 0xFFFFFFFFu;
        if (info == PF_SLOT_HOLE) {
            // the token's shared row, unused: a valid token index, weight 0
            const uint32_t q = S.rg[E1 - 1] + (uint32_t)t;
            b.sorted_tok[q] = (uint16_t)t;
            b.sorted_w[q] = 0.0f;
        } else if (info != 0xFFFFFFFFu) {
            const uint32_t e = info >> PF_SLOT_RANK_BITS, k = (info >> PF_SLOT_COPY_SHIFT) & (PF_CNT_COPIES - 1u);
            p = S.rg[e] + (e < (uint32_t)E1 - 1u ? cb[k * E1 + e] : 0u) + (info & ((1u << PF_SLOT_COPY_SHIFT) - 1u));
            b.sorted_tok[p] = (uint16_t)t;
            b.sorted_w[p] = wv;
        }
        b.pos[i] = p;
    }
}

// ---------------------------------------------------------------- shared pipeline pieces
// A wave-uniform pointer moved to SGPRs (loads then take a scalar base and a lane offset).
template <typename T>
__device__ __forceinline__ const T *uniform_ptr(const T *p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const T *)(((uint64_t)hi << 32) | lo);
}

// Raw IQ4_XS data of one K stage (PF_KC = 128 K = 4 sub-blocks, half a super-block) for NR
// 16-row weight groups, read from the split layout (k_repack_split): lane (g, n) gets the
// header of row n and, in one 16-byte load, the 16 qs bytes of sub-block 4h + g of row n (h =
// the stage's half of the super-block).  MFMA K-step ks of the stage then takes dword ks of
// every lane's sub-block: lane group g supplies K positions 32 g + 8 ks .. + 7 of the stage (in
// the 32-block permuted K order of xh), and its sub-block scale is the same in all 4 steps.
// Stages live in a ring so each is requested a few stages ahead.
struct WRows {
    const uint8_t *q; // qs of the group's first row (matrix base + row * SBR * 128)
    const uint8_t *h; // header of the group's first row (header array + row * SBR * 8)
};

// Rows row0 .. row0 + 15 of a split matrix of `rows` rows and SBR super-blocks per row.
template <int SBR>
__device__ __forceinline__ WRows split_rows(const uint8_t *m, int rows, int row0) {
    return WRows{uniform_ptr(m + (size_t)row0 * SBR * 128),
                 uniform_ptr(m + (size_t)rows * SBR * 128 + (size_t)row0 * SBR * 8)};
}

template <int NR>
struct WStage {
    u32x2 hdr[NR];
    u32x4 q[NR];
};

template <int SBR, int NR>
__device__ __forceinline__ void wstage_load(WStage<NR> &s, const WRows (&groups)[NR], int ch, int lane) {
    const int sb = ch >> 1, h = ch & 1;
    // unsigned lane offsets (zero-extended) on wave-uniform bases that go through
    // readfirstlane: the loads then take an SGPR base and one 32-bit lane offset
    const uint32_t n = (uint32_t)(lane & 15), g = (uint32_t)(lane >> 4);
    const uint32_t oh = n * (SBR * 8u), oq = n * (SBR * 128u) + 16u * g;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        s.hdr[r] = ldg<u32x2>(uniform_ptr(groups[r].h + (size_t)sb * 8) + oh);
        s.q[r] = ldg<u32x4>(uniform_ptr(groups[r].q + (size_t)sb * 128 + 64 * h) + oq);
    }
}

// B and C pairs of the lane's sub-block (4h + g of the stage's super-block) for each row group.
template <int NR>
__device__ __forceinline__ void wstage_bc(const WStage<NR> &s, int ch, int g, const float (&F)[NR],
                                          uint32_t (&b2)[NR], uint32_t (&c2)[NR]) {
#pragma unroll
    for (int r = 0; r < NR; ++r) bc_pair(s.hdr[r], 4 * (ch & 1) + g, F[r], b2[r], c2[r]);
}

// Row shift s_n of weight row n (lane (g, n)): with the row's largest |d| < 2^e (over its SBR
// super-blocks), s_n = e + 13, so every sub-block's |B| = |d (ls - 32)| 2^(24 - s_n) <
// 32 * 2^e * 2^(11 - e) = 2^16, i.e. at most 65504 after rounding (a row's largest |d| times 32
// is an f16 significand times a power of two).  Lane (g, n) requests the d words of a share of
// the row's headers (row_dmax_load, issued with the first loads of the work item); row_shift
// takes the maximum over the row's four lane groups and returns F = 2^(24 - s_n) for bc_pair
// and P = 2^s_n for the epilogue.  A row whose d are all zero gets F = 2^127 (its B are 0).
template <int SBR>
__device__ __forceinline__ u32x2 row_dmax_load(const WRows &w, int n, int g) {
    if constexpr (SBR == 1) {
        return u32x2{ldg<uint32_t>(w.h + (uint32_t)n * 8u), 0u};
    } else {
        static_assert(SBR == 2 || SBR == 4 || SBR == 8, "one or two headers per lane group");
        const u32x4 v = ldg<u32x4>(w.h + (uint32_t)n * (SBR * 8u) + 16u * (uint32_t)(g % (SBR / 2)));
        return u32x2{v[0], v[2]};
    }
}
__device__ __forceinline__ void row_shift(u32x2 d2, float &F, float &P) {
    uint32_t m = (d2[0] & 0x7FFFu) > (d2[1] & 0x7FFFu) ? (d2[0] & 0x7FFFu) : (d2[1] & 0x7FFFu);
    uint32_t o = (uint32_t)__shfl_xor((int)m, 16);
    m = o > m ? o : m;
    o = (uint32_t)__shfl_xor((int)m, 32);
    m = o > m ? o : m;
    const uint32_t eb = __builtin_bit_cast(uint32_t, f16_bits_to_f32(m)) >> 23; // max|d| < 2^(eb - 126)
    const uint32_t fe = 264u - eb, pe = eb + 14u;                               // 127 + 11 - e, 127 + e + 13
    F = __builtin_bit_cast(float, (fe < 254u ? fe : 254u) << 23);
    P = __builtin_bit_cast(float, (pe < 254u ? pe : 254u) << 23);
}

// One stage of MFMAs: NR B fragments (dequantized here) against the MT M-tiles of the LDS
// A chunk.  Each K-step first issues the reads of two A fragments, then the decode VALU work
// (which covers their LDS latency), then the MFMAs, reading the next A fragment two M-tiles
// ahead (A fragments are held two at a time, not MT at a time: fewer live registers).
template <int NR, int MT, int LK>
__device__ __forceinline__ void stage_mfma(const WStage<NR> &s0, const uint32_t (&b2)[NR], const uint32_t (&c2)[NR],
                                           const _Float16 *As, int n, int g, f32x4 (&acc)[MT][NR]) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const _Float16 *ap = As + n * LK + 32 * g + 8 * ks;
        u32x4 av[2];
#pragma unroll
        for (int mt = 0; mt < (MT < 2 ? MT : 2); ++mt) av[mt] = *reinterpret_cast<const u32x4 *>(ap + 16 * mt * LK);
        u32x4 b[NR];
#pragma unroll
        for (int r = 0; r < NR; ++r) b[r] = dq8_f16(s0.q[r][ks], b2[r], c2[r]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const u32x4 cur = av[mt & 1];
            if (mt + 2 < MT) av[mt & 1] = *reinterpret_cast<const u32x4 *>(ap + 16 * (mt + 2) * LK);
#pragma unroll
            for (int r = 0; r < NR; ++r) acc[mt][r] = mfma16(cur, b[r], acc[mt][r]);
        }
    }
}

// ---------------------------------------------------------------- K loop
// A (the tile's token rows, f16) is resident in LDS one chunk at a time -- 64 KB: all of K for
// 16-row tiles, 1024 K for 32 rows, 512 K for 64 rows: every thread helps stage a chunk, one
// barrier, then the 8 waves run the chunk's stages with no barrier inside -- each wave waits
// only for its own weight loads, and the other workgroup on the CU hides the chunk
// boundaries.  Weights come through a per-wave ring
// of 4 register stages, each requested three stages ahead in the order they are consumed (a
// wave's in-order vmcnt waits then never hold a use behind a later prefetch); the ring runs
// on across chunks.  Fully unrolled: with a rolled loop the compiler's vmcnt bookkeeping
// merges at the loop head and waits for every prefetch in flight.
// Stages per resident chunk for MT M-tiles (16*MT rows x KCH*PF_KC halves = 64 KB), and the
// chunk's LDS row stride in halves: +16 B per row, so the 16 rows of an A fragment read hit
// 16 different bank groups.
template <int NCH, int MT>
constexpr int pf_kch() { return NCH < 16 / MT ? NCH : 16 / MT; }
template <int NCH, int MT>
constexpr int pf_ldsr() { return pf_kch<NCH, MT>() * PF_KC + 8; }
constexpr int PF_AS_HALVES = PF_BM * (4 * PF_KC + 8); // the largest chunk (64 rows x 520)

// f(integral_constant<int, 0>) ... f(integral_constant<int, N-1>), in order.
template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, Is...>) {
    (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Waves w and w + 4 of a workgroup share a SIMD; with equal priority the older one runs ahead
// and the younger finishes its K loop alone.  Alternating their priorities stage by stage (sp =
// (w >> 2) & 1) keeps the two abreast: gate/up 1.5-2.5 % faster at configs 1 and 4 (rocprofv3,
// A/B in one call); neutral in the down kernel's four-stage loop, which leaves it out (sp < 0).
__device__ __forceinline__ void alt_prio(int sp, int st) {
    if (sp < 0) return;
    if ((sp ^ st) & 1) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
}

// Weight ring of RD register stages: the prologue requests stages 0..RD-2.
template <int NCH, int RD, int SBR, int NR>
__device__ __forceinline__ void wring_prologue(WStage<NR> (&ws)[RD], const WRows (&rows)[NR], int lane) {
#pragma unroll
    for (int c = 0; c < RD - 1; ++c) {
        if (c < NCH) wstage_load<SBR>(ws[c], rows, c, lane);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// stage_a(c) moves chunk c of A into LDS; chunk 0 is expected in LDS on entry (its loads were
// issued before the weight ring's, so waiting for them did not wait for the weights).
template <int NCH, int RD, int SBR, int NR, int MT, typename StageA>
__device__ __forceinline__ void gemm_resident(WStage<NR> (&ws)[RD], const WRows (&rows)[NR], const float (&F)[NR],
                                              const _Float16 *As, int n, int g, int sp, f32x4 (&acc)[MT][NR],
                                              StageA stage_a) {
    constexpr int KCH = pf_kch<NCH, MT>();
    constexpr int LK = pf_ldsr<NCH, MT>();
    static_assert(NCH % KCH == 0 && 16 * MT * LK <= PF_AS_HALVES, "whole chunks that fit");
    static_for<NCH>([&](auto CHc) __attribute__((always_inline)) {
        constexpr int ch = decltype(CHc)::value, S = ch % RD;
        if constexpr (ch > 0 && ch % KCH == 0) {
            lds_barrier(); // every wave is done with the previous chunk
            stage_a(ch / KCH);
            lds_barrier();
        }
        alt_prio(sp, ch);
        uint32_t b2[NR], c2[NR];
        wstage_bc(ws[S], ch, g, F, b2, c2);
        stage_mfma<NR, MT, LK>(ws[S], b2, c2, As + (ch % KCH) * PF_KC, n, g, acc);
        // keep the scheduler from moving loads across stages: each stage's weights are
        // requested RD-1 stages ahead, in the order they are consumed
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (ch + RD - 1 < NCH) wstage_load<SBR>(ws[(ch + RD - 1) % RD], rows, ch + RD - 1, n + 16 * g);
        __builtin_amdgcn_sched_barrier(0);
    });
}

// The same K loop with the stages split between two waves: the wave of parity p runs stages
// 2c + p (half super-block p of super-block c), so each decodes half the weights of its
// columns; chunk boundaries (KCH even) fall at the same loop index for both.  Half-length
// work items: gate/up's items then fill the 512 workgroup slots in three rounds of half
// length instead of two full ones (at M = 512, ~1140 items against ~570 of twice the length).
template <int NCH, int RD, int SBR, int NR, int MT, typename StageA>
__device__ __forceinline__ void gemm_resident_split(WStage<NR> (&ws)[RD], const WRows (&rows)[NR],
                                                    const float (&F)[NR], const _Float16 *As, int n, int g,
                                                    int p, f32x4 (&acc)[MT][NR], StageA stage_a) {
    constexpr int KCH = pf_kch<NCH, MT>();
    constexpr int LK = pf_ldsr<NCH, MT>();
    constexpr int NC2 = NCH / 2;
    static_assert(NCH % KCH == 0 && KCH % 2 == 0 && 16 * MT * LK <= PF_AS_HALVES, "whole chunks of even length");
    static_for<NC2>([&](auto Cc) __attribute__((always_inline)) {
        constexpr int c = decltype(Cc)::value, S = c % RD, ch0 = 2 * c;
        if constexpr (ch0 > 0 && ch0 % KCH == 0) {
            lds_barrier();
            stage_a(ch0 / KCH);
            lds_barrier();
        }
        const int ch = ch0 + p;
        alt_prio(p, c);
        uint32_t b2[NR], c2[NR];
        wstage_bc(ws[S], ch, g, F, b2, c2);
        stage_mfma<NR, MT, LK>(ws[S], b2, c2, As + (ch0 % KCH + p) * PF_KC, n, g, acc);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (c + RD - 1 < NC2) wstage_load<SBR>(ws[(c + RD - 1) % RD], rows, 2 * (c + RD - 1) + p, n + 16 * g);
        __builtin_amdgcn_sched_barrier(0);
    });
}

// A tile holds up to PF_BM slots of one expert and runs as 1, 2 or 4 M-tiles of 16 rows (one
// instantiation each, picked per workgroup, so every inner loop is straight-line code).  Full
// PF_BM tiles come first in the list, remainders after: the long work items start first and
// the short ones fill in.  64-row tiles, not 128: every wave reads each A fragment from LDS
// once per pair of B fragments, so LDS traffic per K step grows with the tile height;
// measured, a 128-row tile took 2.5x the time of a 64-row one, more than the second decode of
// the weights that two 64-row tiles cost.
template <typename F>
__device__ __forceinline__ void by_mtiles(int nrows, F f) {
    static_assert(PF_BM == 64 && PF_SMALL_MAX == 32, "tile classes");
    if (nrows > PF_SMALL_MAX) f(std::integral_constant<int, 4>{});
    else if (nrows > 16) f(std::integral_constant<int, 2>{});
    else f(std::integral_constant<int, 1>{});
}

// The (tile, item) of this workgroup in a launch of ITEMS x T workgroups (T a multiple of 8,
// tiles past a.tile_max exit).  GROUP: the hardware hands linear workgroup w = x + ITEMS y to
// XCD w % 8, so tile 8 (k / ITEMS) + w % 8, item k % ITEMS (k = w / 8) puts every item of a
// tile on one XCD -- the tile's token rows (gate/up) or h rows (down) come from HBM once and
// are L2 hits for its other items -- and consecutive tiles on consecutive XCDs, in dispatch
// order.  Used for the wide items of large M (measured, M = 4096: gate/up 310 -> 292 us, down
// 189 -> 176 us); at M <= 768 the rows of all the tiles stay in the memory-side cache anyway
// and one tile's items spread over the eight XCDs run faster (M = 512: 124 against 132 us).
template <int ITEMS, bool GROUP>
__device__ __forceinline__ void xcd_tile_item(int &tile, int &item) {
    if constexpr (GROUP) {
        const int w = (int)blockIdx.x + ITEMS * (int)blockIdx.y, k = w >> 3;
        tile = 8 * (k / ITEMS) + (w & 7);
        item = k % ITEMS;
    } else {
        tile = (int)blockIdx.y;
        item = (int)blockIdx.x;
    }
}

// ---------------------------------------------------------------- gate/up
// SPLIT: PF_NGU columns per item, two waves per 16 columns on alternate stages; else
// PF_NGU_WIDE columns, one wave per 16 columns on every stage.
// Kernel arguments a work item's chain needs, fetched at the kernel's first instructions: one
// asm takes them all as inputs, so the compiler loads them in one batch of scalar loads (the
// values and the pointers' address space unchanged) instead of one at a time at each first use
// -- the tile list, then the token ids, then the layer's pointers, then the A rows' base, each
// with its own wait between the tile record and the first A load.
__device__ __forceinline__ void fetch_gate_up_args(const PrefillArgs &a) {
    asm volatile("" ::"s"(a.tiles), "s"(a.tile_max), "s"(a.sorted_tok), "s"(a.xinv), "s"(a.xh), "s"(a.L.w1),
                 "s"(a.L.w3), "s"(a.L.s1), "s"(a.L.s3), "s"(a.L.sw1), "s"(a.L.sw3), "s"(a.E), "s"(a.hh), "s"(a.hmax));
}
__device__ __forceinline__ void fetch_down_args(const PrefillArgs &a) {
    asm volatile("" ::"s"(a.tiles), "s"(a.tile_max), "s"(a.L.w2), "s"(a.L.s2), "s"(a.L.sw2), "s"(a.E), "s"(a.hh),
                 "s"(a.hmax), "s"(a.sorted_w), "s"(a.c), "s"(a.part), "s"(a.pexp));
}

// A tile record in one 16-byte load (read field by field, the compiler fetched the expert, tested
// it, and only then fetched row0 and nrows: one more round trip before the A rows).
__device__ __forceinline__ Tile tile_record(const Tile *tiles, int ti) {
    const u32x4 v = ldg<u32x4>(tiles + ti);
    return Tile{(int32_t)v[0], (int32_t)v[1], (int32_t)v[2], 0};
}

template <int H, int I, bool SPLIT>
__global__ __launch_bounds__(64 * PF_WAVES, 4) void k_pf_gate_up(PrefillArgs a) {
    constexpr int NGU = SPLIT ? PF_NGU : PF_NGU_WIDE;
    static_assert(NGU == 16 * PF_WAVES / (SPLIT ? 2 : 1), "16 columns per wave (pair)");
    constexpr int NCH = H / PF_KC;
    constexpr int SBR = H / QK;
    static_assert(H % QK == 0 && I % NGU == 0 && PF_KC * 2 == QK, "gate/up shape");
    __shared__ __attribute__((aligned(16))) _Float16 As[PF_AS_HALVES];
    __shared__ uint32_t rowmax[PF_BM];
    __shared__ float s_inv[PF_BM];
    __shared__ int s_tok[PF_BM];
    fetch_gate_up_args(a);

    int ti, item;
    xcd_tile_item<I / NGU, !SPLIT>(ti, item);
    if (ti >= a.tile_max) return;
    const Tile tl = tile_record(a.tiles, ti);
    if (tl.expert < 0) return;
    const int e = tl.expert, row0 = tl.row0, nrows = tl.nrows;
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6); // wave-uniform (SGPR)
    const int n = lane & 15, g = lane >> 4;
    const int cw = SPLIT ? (wv & 3) : wv, p = SPLIT ? (wv >> 2) : 0; // column group, stage parity
    const int c0 = item * NGU + cw * 16; // this wave's h columns
    // the tile's tokens (rows past nrows repeat the last token); their 1/scale is requested
    // here but only waited for, and put in LDS, before the epilogue: A's loads depend on the
    // tokens, not on it
    float inv_t = 0.0f;
    if (tid < PF_BM) {
        const int t = a.sorted_tok[row0 + (tid < nrows ? tid : nrows - 1)];
        s_tok[tid] = t;
        rowmax[tid] = 0u;
        inv_t = a.xinv[t];
    }
    lds_barrier();
    // Weights: rows c0 + n of W1 (gate) and W3 (up).
    const WRows rows[2] = {split_rows<SBR>(expert_w(a.L.w1, a.L.s1, a.L.sw1, e, a.E), I, c0),
                           split_rows<SBR>(expert_w(a.L.w3, a.L.s3, a.L.sw3, e, a.E), I, c0)};

    by_mtiles(nrows, [&](auto MTc) __attribute__((always_inline)) {
        constexpr int MT = decltype(MTc)::value;
        constexpr int KC = pf_kch<NCH, MT>() * PF_KC, LK = pf_ldsr<NCH, MT>();
        // chunk c of A: 16*MT rows x KC halves, 16 B per lane, a row spanning whole waves
        constexpr int QPR = KC / 8, PER = 16 * MT * QPR / (64 * PF_WAVES);
        static_assert(PER >= 1 && 16 * MT * QPR % (64 * PF_WAVES) == 0 && QPR % 64 == 0, "A staging split");
        u32x4 va[PER];
        // quads [i0, i1) of chunk c: global -> registers, registers -> LDS
        auto load_a = [&](int c, int i0, int i1) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < PER; ++i)
                if (i >= i0 && i < i1) {
                    const int idx = i * 64 * PF_WAVES + tid, r = idx / QPR, q = idx % QPR;
                    // r is the same for the whole wave (QPR % 64 == 0): the row base in SGPRs
                    const int tok = __builtin_amdgcn_readfirstlane(s_tok[r]);
                    const _Float16 *rowp = uniform_ptr(a.xh + (size_t)tok * H + c * KC);
                    va[i] = ldg<u32x4>(rowp + 8u * (uint32_t)q);
                }
        };
        auto store_a = [&](int i0, int i1) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < PER; ++i)
                if (i >= i0 && i < i1) {
                    const int idx = i * 64 * PF_WAVES + tid, r = idx / QPR, q = idx % QPR;
                    *reinterpret_cast<u32x4 *>(As + r * LK + 8 * q) = va[i];
                }
        };
        constexpr int RD = 3; // weight ring depth: two stages ahead (register budget)
        WStage<2> ws[RD];
        load_a(0, 0, PER);
        // the rows' headers for their shifts after A and before the first weights (requested
        // ahead of A, their registers were reused by A's addressing and the A loads waited for
        // them; requested after the weights, the first stage would wait for all of those)
        const u32x2 dq[2] = {row_dmax_load<SBR>(rows[0], n, g), row_dmax_load<SBR>(rows[1], n, g)};
        if constexpr (SPLIT) {
#pragma unroll
            for (int c = 0; c < RD - 1; ++c) {
                if (c < NCH / 2) wstage_load<SBR>(ws[c], rows, 2 * c + p, lane);
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
            wring_prologue<NCH, RD, SBR>(ws, rows, lane);
        }
        store_a(0, PER);
        float F[2], P[2];
        row_shift(dq[0], F[0], P[0]);
        row_shift(dq[1], F[1], P[1]);
        lds_barrier();
        f32x4 acc[MT][2];
#pragma unroll
        for (int i = 0; i < MT; ++i) acc[i][0] = acc[i][1] = f32x4{0, 0, 0, 0};
        // later chunks are moved in two halves while the weight ring and the accumulators
        // are live (fewer registers held at once)
        constexpr int HALF = (PER + 1) / 2;
        auto stage_a = [&](int c) __attribute__((always_inline)) {
            load_a(c, 0, HALF);
            store_a(0, HALF);
            load_a(c, HALF, PER);
            store_a(HALF, PER);
        };
        if (tid < PF_BM) s_inv[tid] = inv_t;
        // the wave's elements: el = 4 mt + i is row 16 mt + 4 g + i of the tile, column c0 + n.
        // With SPLIT the two partner waves (stage parities 0 and 1) each finish half of them:
        // parity 0 elements el < NE/2, parity 1 the rest, after handing each other the partial
        // sums of the partner's half through the (then free) A chunk.
        constexpr int NE = 4 * MT, NOWN = SPLIT ? NE / 2 : NE;
        const int el0 = SPLIT && p ? NE / 2 : 0;
        if constexpr (SPLIT) {
            gemm_resident_split<NCH, RD, SBR, 2, MT>(ws, rows, F, As, n, g, p, acc, stage_a);
            __builtin_amdgcn_s_setprio(0);
            lds_barrier();
            float *red = reinterpret_cast<float *>(As);
            static_assert(4 * NE * 2 * 64 * 4 <= PF_AS_HALVES * 2, "the pair sums fit the A chunk");
#pragma unroll
            for (int el = 0; el < NE; ++el)
                if ((el < NE / 2) == (p != 0))
#pragma unroll
                    for (int r = 0; r < 2; ++r) red[((cw * NE + el) * 2 + r) * 64 + lane] = acc[el / 4][r][el % 4];
            lds_barrier();
#pragma unroll
            for (int el = 0; el < NE; ++el)
                if ((el < NE / 2) == (p == 0))
#pragma unroll
                    for (int r = 0; r < 2; ++r) acc[el / 4][r][el % 4] += red[((cw * NE + el) * 2 + r) * 64 + lane];
        } else {
            gemm_resident<NCH, RD, SBR, 2, MT>(ws, rows, F, As, n, g, (wv >> 2) & 1, acc, stage_a);
            __builtin_amdgcn_s_setprio(0);
            lds_barrier(); // s_inv
        }

        // epilogue: h = silu(g) * u with the token scale and the row shifts undone; per-row max|h| of the item's
        // columns, then h as f16 scaled by the power of two that puts that max in [2^14, 2^15),
        // stored in the down kernel's K order (perm32_pos inside every 32-column block)
        float hv[NOWN];
#pragma unroll
        for (int j = 0; j < NOWN; ++j) {
            const int el = el0 + j, m = 16 * (el / 4) + 4 * g + el % 4;
            // element j of this wave's half (selected, not indexed: acc stays in registers)
            constexpr int JH = SPLIT ? NE / 2 : 0;
            const float gv = SPLIT && p ? acc[(JH + j) / 4][0][(JH + j) % 4] : acc[j / 4][0][j % 4];
            const float uv = SPLIT && p ? acc[(JH + j) / 4][1][(JH + j) % 4] : acc[j / 4][1][j % 4];
            hv[j] = 0.0f;
            if (m < nrows) {
                const float inv = s_inv[m];
                hv[j] = silu_rcp(gv * (P[0] * inv)) * (uv * (P[1] * inv));
            }
            const float rm = max16(fabsf(hv[j]));
            if (n == 0) atomicMax(&rowmax[m], __builtin_bit_cast(uint32_t, rm));
        }
        lds_barrier();
        const int col = c0 + n, hcol = (col & ~31) + perm32_pos(col & 31);
#pragma unroll
        for (int j = 0; j < NOWN; ++j) {
            const int el = el0 + j, m = 16 * (el / 4) + 4 * g + el % 4;
            if (m < nrows) {
                float unused;
                const float sc = pow2_scale(__builtin_bit_cast(float, rowmax[m]), &unused);
                a.hh[(uint32_t)((row0 + m) * I + hcol)] = (_Float16)(hv[j] * sc); // < 2^31: 9 m_max I
            }
        }
    });
    if (tid < nrows) a.hmax[(size_t)(row0 + tid) * (I / NGU) + item] = __builtin_bit_cast(float, rowmax[tid]);
}

// ---------------------------------------------------------------- down
// NGU: the column width of h's scale blocks (the gate/up item width).
template <int H, int I, int NGU>
__global__ __launch_bounds__(64 * PF_WAVES, 4) void k_pf_down(PrefillArgs a) {
    constexpr int NTW = 2, NCH = I / PF_KC;
    constexpr int SBR = I / QK;
    constexpr int NHB = I / NGU; // h max blocks per row
    constexpr int BPR = I / 32;      // 32-blocks per row
    static_assert(I % QK == 0 && H % PF_ND == 0 && PF_KC * 2 == QK, "down shape");
    static_assert(pf_kch<NCH, 4>() == NCH, "all of K = inter resident in one chunk");
    __shared__ __attribute__((aligned(16))) _Float16 As[PF_AS_HALVES];
    __shared__ float s_sc[PF_BM];
    fetch_down_args(a);

    int ti, item;
    xcd_tile_item<H / PF_ND, NGU == PF_NGU_WIDE>(ti, item);
    if (ti >= a.tile_max) return;
    const Tile tl = tile_record(a.tiles, ti);
    if (tl.expert < 0) return;
    const int e = tl.expert, row0 = tl.row0, nrows = tl.nrows;
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6); // wave-uniform (SGPR)
    const int n = lane & 15, g = lane >> 4;
    const int r0 = item * PF_ND + wv * 32; // this wave's output rows r0 .. r0+31
    const uint8_t *w2 = expert_w(a.L.w2, a.L.s2, a.L.sw2, e, a.E);
    const WRows rows[NTW] = {split_rows<SBR>(w2, H, r0), split_rows<SBR>(w2, H, r0 + 16)};

    by_mtiles(nrows, [&](auto MTc) __attribute__((always_inline)) {
        constexpr int MT = decltype(MTc)::value;
        constexpr int LK = pf_ldsr<NCH, MT>();
        // A: 16*MT rows x BPR 32-blocks; a thread takes blocks tid, tid + 512, ... -- each one
        // 32 f16 of h, already in the weights' K order and scaled by its NGU-column block's
        // power of two; rescaled here to the power of two of the row's max (a factor 2^-j,
        // exact for normal f16).  All loads (h and the row's max blocks) are issued before any
        // is used.
        constexpr int NIT = 16 * MT * BPR, IPT = (NIT + 64 * PF_WAVES - 1) / (64 * PF_WAVES);
        static_assert(NGU % 32 == 0, "max blocks of whole 32-blocks");
        u32x4 hq[IPT][4];
        float hm[IPT][NHB], sw[IPT];
#pragma unroll
        for (int j = 0; j < IPT; ++j) {
            const int it = j * 64 * PF_WAVES + tid;
            if (IPT * 64 * PF_WAVES == NIT || it < NIT) {
                const int ar = it / BPR, ab = it % BPR;
                const int slot = row0 + (ar < nrows ? ar : nrows - 1);
                const u32x4 *src = reinterpret_cast<const u32x4 *>(a.hh + (size_t)slot * I + 32 * ab);
#pragma unroll
                for (int i = 0; i < 4; ++i) hq[j][i] = ldg<u32x4>(src + i);
#pragma unroll
                for (int b = 0; b < NHB; ++b) hm[j][b] = a.hmax[(size_t)slot * NHB + b];
                // the slot's weight, for the epilogue (loaded with the h rows, not after the GEMM)
                sw[j] = ab == 0 ? a.sorted_w[slot] : 0.0f;
            }
        }
        // the rows' headers for their shifts after the h rows, before the weights (requested
        // first, their registers were reused by the h rows' addressing and the h loads waited)
        const u32x2 dq[NTW] = {row_dmax_load<SBR>(rows[0], n, g), row_dmax_load<SBR>(rows[1], n, g)};
        constexpr int RD = 4; // weight ring depth: three stages ahead
        WStage<NTW> ws[RD];
        wring_prologue<NCH, RD, SBR>(ws, rows, lane);
#pragma unroll
        for (int j = 0; j < IPT; ++j) {
            const int it = j * 64 * PF_WAVES + tid;
            if (IPT * 64 * PF_WAVES == NIT || it < NIT) {
                const int ar = it / BPR, ab = it % BPR;
                float mx = 0.f;
#pragma unroll
                for (int b = 0; b < NHB; ++b) mx = fmaxf(mx, hm[j][b]);
                float inv, inv_b;
                const float sc = pow2_scale(ar < nrows ? mx : 0.0f, &inv);
                const float hb = hm[j][ab / (NGU / 32)];
                (void)pow2_scale(hb, &inv_b);
                if (ab == 0) s_sc[ar] = ar < nrows ? a.c * sw[j] * inv : 0.0f; // the row's epilogue factor
                // 2^-j, j >= 0, for a block with a nonzero max; a block whose max is 0 holds
                // only zeros, and its factor is 0 (sc alone can exceed the f16 range when the
                // row's max is small: 0 * inf would be NaN)
                const _Float16 f = hb > 0.0f ? (_Float16)(sc * inv_b) : (_Float16)0.0f;
                const f16x2 f2 = {f, f};
                u32x4 *d = reinterpret_cast<u32x4 *>(As + ar * LK + 32 * ab);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const u32x4 q4 = hq[j][i];
                    u32x4 o;
#pragma unroll
                    for (int e = 0; e < 4; ++e) o[e] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, (uint32_t)q4[e]) * f2);
                    d[i] = o;
                }
            }
        }
        float F[NTW], P[NTW];
#pragma unroll
        for (int t = 0; t < NTW; ++t) row_shift(dq[t], F[t], P[t]);
        lds_barrier();
        f32x4 acc[MT][NTW];
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int t = 0; t < NTW; ++t) acc[i][t] = f32x4{0, 0, 0, 0};
        gemm_resident<NCH, RD, SBR, NTW, MT>(ws, rows, F, As, n, g, -1, acc, [](int) {});

        // epilogue: v = c * w * 2^-s_row * 2^s_n * acc per slot row (s_n: the weight row's shift); each row's 32 values of this
        // wave are stored as f16 times a power of two 2^sh that puts their max in
        // [2^14, 2^15), sh kept beside them (one byte per row and 32 columns), column n and
        // 16 + n of the block side by side (stored position 2n, 2n + 1).  Through LDS
        // (As is free once every wave is done with it) so that each lane stores whole 16-byte
        // row pieces.
        static_assert(PF_WAVES * PF_BM * 32 * 2 <= PF_AS_HALVES * 2, "transpose fits in As");
        lds_barrier();
        _Float16 *T = As + wv * (16 * MT * 32); // [16 MT rows][32 columns]
        const int cb = r0 / 32;                 // this wave's 32-column block
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = 16 * mt + 4 * g + i;
                const float sc = s_sc[m]; // c * w * 2^-s_row (0 past nrows)
                float v[NTW], mx = 0.0f;
#pragma unroll
                for (int t = 0; t < NTW; ++t) {
                    v[t] = sc * (P[t] * acc[mt][t][i]);
                    mx = fmaxf(mx, fabsf(v[t]));
                }
                mx = max16(mx); // the row's 32 columns: 16 lanes x NTW
                const int sh = pow2_shift(mx);
                static_assert(NTW == 2, "columns n and 16 + n of a block stored as one f16 pair");
                *reinterpret_cast<uint32_t *>(T + m * 32 + 2 * n) =
                    pack_f16x2(__builtin_amdgcn_ldexpf(v[0], sh), __builtin_amdgcn_ldexpf(v[1], sh));
                if (n == 0 && m < nrows) a.pexp[(size_t)(row0 + m) * (H / 32) + cb] = (int8_t)sh;
            }
        // lanes read what other lanes of this wave wrote: LDS keeps a wave's accesses in
        // order, the compiler must too
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int k = lane; k < 16 * MT * 4; k += 64) {
            const int r = k >> 2, q = k & 3;
            if (r < nrows)
                *reinterpret_cast<u32x4 *>(a.part + (size_t)(row0 + r) * H + r0 + 8 * q) =
                    *reinterpret_cast<const u32x4 *>(T + r * 32 + 8 * q);
        }
    });
}

// ---------------------------------------------------------------- combine
// y_t (+)= sum_{s=0..8} part[pos[t][s]] * 2^-pexp; restates the weighted sum that the
// reference's w2_scatter epilogue accumulates into the hidden state
// (shaders/w2_scatter.comp:77-86), in a fixed order, in f32.  A thread owns 8 stored f16:
// in 32-column block b, pairs j = 4 (c8 % 4) .. + 3, i.e. columns 32 b + j and 32 b + 16 + j.
template <int H>
__global__ __launch_bounds__(256) void k_pf_combine(PrefillArgs a) {
    const int t = blockIdx.x;
    // the chain's bucket counters, read by k_pf_place (an earlier launch), start over at zero
    if (t == 0 && a.cnt)
        for (int e = threadIdx.x; e < PF_CNT_COPIES * (a.E + 1); e += 256) a.cnt[e] = 0u;
    uint32_t ps[SLOTS];
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) ps[s] = a.pos[(size_t)t * SLOTS + s];
    for (int c8 = threadIdx.x; c8 < H / 8; c8 += 256) {
        u32x4 q[SLOTS];
        float f[SLOTS];
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) { // all loads first; a dropped slot loads row 0, unused
            const uint32_t p = ps[s] != 0xFFFFFFFFu ? ps[s] : 0u;
            q[s] = ldg<u32x4>(a.part + (size_t)p * H + 8 * c8);
            f[s] = __builtin_amdgcn_ldexpf(1.0f, -(int)a.pexp[(size_t)p * (H / 32) + c8 / 4]);
        }
        f32x4 lo = {0, 0, 0, 0}, hi = {0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) {
            // a dropped slot adds nothing (not 0 times row 0, which may be non-finite or stale)
            const bool on = ps[s] != 0xFFFFFFFFu;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const f16x2 h2 = __builtin_bit_cast(f16x2, (uint32_t)q[s][j]);
                lo[j] = on ? lo[j] + (float)h2[0] * f[s] : lo[j];
                hi[j] = on ? hi[j] + (float)h2[1] * f[s] : hi[j];
            }
        }
        float *yb = a.y + (size_t)t * H + 32 * (c8 / 4) + 4 * (c8 % 4);
        f32x4 *y0 = reinterpret_cast<f32x4 *>(yb), *y1 = reinterpret_cast<f32x4 *>(yb + 16);
        const f32x4 b0 = a.accumulate ? *y0 : f32x4{0, 0, 0, 0};
        const f32x4 b1 = a.accumulate ? *y1 : f32x4{0, 0, 0, 0};
        *y0 = b0 + lo;
        *y1 = b1 + hi;
    }
}

template <int H, int I>
static hipError_t launch_prefill_t(const BucketArgs &b, const PfCountArgs &c, const PrefillArgs &a, hipStream_t st,
                                   KernelTimer *T) {
    // the chain's own fill: count (routing first with logits), then place + prep
    {
        TimedLaunch tl(T, c.logits ? MOE_K_ROUTER_TOPK : MOE_K_BUCKET_FILL, st);
        const dim3 grid((unsigned)((c.M + PF_COUNT_TOKENS - 1) / PF_COUNT_TOKENS));
        if (c.logits) hipLaunchKernelGGL(k_pf_count<true>, grid, dim3(64 * PF_COUNT_TOKENS), 0, st, c);
        else hipLaunchKernelGGL(k_pf_count<false>, grid, dim3(64 * PF_COUNT_TOKENS), 0, st, c);
    }
    {
        TimedLaunch tl(T, MOE_K_BUCKET_FILL, st);
        const int nplace = (SLOTS * b.M + PF_PLACE_SLOTS - 1) / PF_PLACE_SLOTS;
        const int nprep = (a.M + PF_PREP_TOKENS - 1) / PF_PREP_TOKENS;
        hipLaunchKernelGGL((k_pf_place<H>), dim3((unsigned)(nplace + nprep)), dim3(BF_THREADS),
                           (5 * (size_t)(b.E1 + 1) + (size_t)PF_CNT_COPIES * b.E1) * 4, st, b, c, a);
    }
    // one launch over the tile list (full and big remainder tiles, then small remainders, then
    // empty entries, which exit at once)
    const int ntiles = (a.tile_max + 7) / 8 * 8; // whole groups of 8 tiles (xcd_tile_item)
    const bool split = a.M <= PF_SPLIT_MAX_M;
    {
        TimedLaunch tl(T, MOE_K_PREFILL_GATE_UP, st);
        if (split) hipLaunchKernelGGL((k_pf_gate_up<H, I, true>), dim3(I / PF_NGU, ntiles), dim3(64 * PF_WAVES), 0, st, a);
        else hipLaunchKernelGGL((k_pf_gate_up<H, I, false>), dim3(I / PF_NGU_WIDE, ntiles), dim3(64 * PF_WAVES), 0, st, a);
    }
    {
        TimedLaunch tl(T, MOE_K_PREFILL_DOWN, st);
        if (split) hipLaunchKernelGGL((k_pf_down<H, I, PF_NGU>), dim3(H / PF_ND, ntiles), dim3(64 * PF_WAVES), 0, st, a);
        else hipLaunchKernelGGL((k_pf_down<H, I, PF_NGU_WIDE>), dim3(H / PF_ND, ntiles), dim3(64 * PF_WAVES), 0, st, a);
    }
    {
        TimedLaunch tl(T, MOE_K_PREFILL_COMBINE, st);
        hipLaunchKernelGGL((k_pf_combine<H>), dim3(a.M), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

hipError_t launch_prefill(int H, int I, const BucketArgs &b, const PfCountArgs &c, const PrefillArgs &a,
                          hipStream_t st, KernelTimer *T) {
    if (H == 2048 && I == 512) return launch_prefill_t<2048, 512>(b, c, a, st, T);
    if (H == 512 && I == 256) return launch_prefill_t<512, 256>(b, c, a, st, T);
    return hipErrorInvalidValue;
}

} // namespace moe
