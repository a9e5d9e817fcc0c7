// k_prefill.hip -- prefill path (M > 8): grouped IQ4_XS-dequant bf16 MFMA GEMMs.
//
// Replaces the reference's bucketed prefill dispatches (src/inference.rs:683-732): per
// non-empty bucket a tiled w1_w3_fused GEMM into an f16 scratch and a w2_scatter GEMM
// whose epilogue read-modify-writes the f16 hidden state (shaders/w1_w3_fused.comp,
// shaders/w2_scatter.comp).  Here, after the bucket fill has produced expert-sorted slots
// and a tile list:
//   prep:    x -> bf16 (RMSNorm fused when asked), once per token;
//   gate_up: per (tile of <=64 slots of one expert, 64 gate/up column pairs) a bf16 MFMA
//            GEMM over K = hidden; the slot rows are gathered from the token rows (the
//            reference's kernel skipped this gather); weight tiles are decoded from IQ4_XS
//            to bf16(d*(ls-32)*kv) straight into LDS; SiLU(gate)*up in the epilogue;
//   down:    per (tile, 64 output columns) the same over K = inter, epilogue scales by
//            c * slot weight and writes one f32 row per slot;
//   combine: y_t (+)= sum over t's 9 slots in slot order -- deterministic, no atomics, no
//            f16 read-modify-write race.
// MFMA: v_mfma_f32_16x16x32_bf16, 4 waves per 64x64 tile, each wave 32x32 (2x2 frags).
#include "moe_internal.hpp"

namespace moe {

constexpr int PF_BK = 128;
constexpr int PF_LDSK = PF_BK + 8; // +16 B per LDS row breaks the 256-B bank period

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    __bf16 l = (__bf16)lo, h = (__bf16)hi;
    return (uint32_t)__builtin_bit_cast(uint16_t, l) | ((uint32_t)__builtin_bit_cast(uint16_t, h) << 16);
}

// One 32-weight sub-block (16 qs bytes) -> 32 bf16(dl * kv) in natural K order, written
// as four 16-byte LDS stores at dst (dst[0..15] = weights 0..15, dst[16..31] = 16..31).
__device__ __forceinline__ void dequant_sub_bf16(u32x4 qs, float dl, __bf16 *dst) {
    u32x4 lo4[2], hi4[2];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        uint32_t lo, hi;
        kv_signed8(qs[w], lo, hi);
        lo4[w >> 1][2 * (w & 1) + 0] = pack_bf16x2(dl * sbyte(lo, 0), dl * sbyte(lo, 1));
        lo4[w >> 1][2 * (w & 1) + 1] = pack_bf16x2(dl * sbyte(lo, 2), dl * sbyte(lo, 3));
        hi4[w >> 1][2 * (w & 1) + 0] = pack_bf16x2(dl * sbyte(hi, 0), dl * sbyte(hi, 1));
        hi4[w >> 1][2 * (w & 1) + 1] = pack_bf16x2(dl * sbyte(hi, 2), dl * sbyte(hi, 3));
    }
    u32x4 *d4 = reinterpret_cast<u32x4 *>(dst);
    d4[0] = lo4[0];
    d4[1] = lo4[1];
    d4[2] = hi4[0];
    d4[3] = hi4[1];
}

__device__ __forceinline__ f32x4 mfma_bf16(const __bf16 *a, const __bf16 *b, f32x4 c) {
    bf16x8 av = *reinterpret_cast<const bf16x8 *>(a);
    bf16x8 bv = *reinterpret_cast<const bf16x8 *>(b);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, c, 0, 0, 0);
}

// ---------------------------------------------------------------- prep
template <int H>
__global__ __launch_bounds__(256) void k_pf_prep(PrefillArgs a) {
    constexpr int PER = H / 256;
    __shared__ float red[4];
    const int t = blockIdx.x, tid = threadIdx.x;
    const float *xr = a.x + (size_t)t * H + tid * PER;
    float v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) v[i] = xr[i];
    float inv = 1.0f;
    if (a.rmsnorm) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < PER; ++i) ss = __builtin_fmaf(v[i], v[i], ss);
        ss = group_sum<64>(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        const float tot = (red[0] + red[1]) + (red[2] + red[3]);
        inv = 1.0f / sqrtf(tot * (1.0f / (float)H) + 1e-6f);
    }
    __bf16 *dst = a.xb + (size_t)t * H + tid * PER;
#pragma unroll
    for (int i = 0; i < PER; ++i) dst[i] = (__bf16)(v[i] * inv);
}

// ---------------------------------------------------------------- gate/up
template <int H, int I>
__global__ __launch_bounds__(256) void k_pf_gate_up(PrefillArgs a) {
    constexpr int BM = PF_BM, BNH = 64, BK = PF_BK, LDSK = PF_LDSK;
    constexpr int ROWB = (H / QK) * SB_BYTES;
    constexpr int NSTEP = H / BK;
    static_assert(H % BK == 0 && I % BNH == 0, "tile shape");
    __shared__ __attribute__((aligned(16))) __bf16 As[BM * LDSK];
    __shared__ __attribute__((aligned(16))) __bf16 Bs[2 * BNH * LDSK];

    const Tile tl = a.tiles[blockIdx.x];
    if (tl.expert < 0) return;
    const int e = tl.expert;
    const int n0 = blockIdx.y * BNH;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;

    // A staging: row am, 32 bf16 at column 32*aq of the K step.
    const int am = tid >> 2, aq = tid & 3;
    const bool arow = am < tl.nrows;
    const int tok = arow ? (int)a.sorted_tok[tl.row0 + am] : 0;
    const __bf16 *asrc = a.xb + (size_t)tok * H + 32 * aq;
    // B staging: weight row br (0..63 gate = W1, 64..127 up = W3), sub-blocks 2*bh, 2*bh+1.
    const int br = tid >> 1, bh = tid & 1;
    const uint8_t *Wb = (br < BNH) ? expert_w(a.L.w1, a.L.s1, a.L.sw1, e, a.E)
                                   : expert_w(a.L.w3, a.L.s3, a.L.sw3, e, a.E);
    const uint8_t *brow = Wb + (size_t)(n0 + (br & (BNH - 1))) * ROWB;

    u32x4 ra[4];
    u32x2 rh;
    u32x4 rq[2];
    auto gload = [&](int step) {
        const int k0 = step * BK;
#pragma unroll
        for (int i = 0; i < 4; ++i) ra[i] = arow ? ldg<u32x4>(asrc + k0 + 8 * i) : u32x4{0, 0, 0, 0};
        const int g0 = k0 / 32 + 2 * bh;
        const uint8_t *sbp = brow + (size_t)(g0 >> 3) * SB_BYTES;
        rh = ldg<u32x2>(sbp);
        rq[0] = ldg<u32x4>(sbp + 8 + 16 * (g0 & 7));
        rq[1] = ldg<u32x4>(sbp + 8 + 16 * ((g0 & 7) + 1));
    };

    f32x4 accg[2][2], accu[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            accg[i][j] = f32x4{0, 0, 0, 0};
            accu[i][j] = f32x4{0, 0, 0, 0};
        }
    const int mh = wv & 1, nh = wv >> 1;
    const int fr = lane & 15, fk = 8 * (lane >> 4);

    gload(0);
    for (int step = 0; step < NSTEP; ++step) {
        {
            u32x4 *ad = reinterpret_cast<u32x4 *>(As + am * LDSK + 32 * aq);
#pragma unroll
            for (int i = 0; i < 4; ++i) ad[i] = ra[i];
            const int g0 = (step * BK) / 32 + 2 * bh;
#pragma unroll
            for (int j = 0; j < 2; ++j)
                dequant_sub_bf16(rq[j], sub_scale(rh, (g0 & 7) + j), Bs + br * LDSK + 64 * bh + 32 * j);
        }
        __syncthreads();
        if (step + 1 < NSTEP) gload(step + 1);
#pragma unroll
        for (int kk = 0; kk < BK / 32; ++kk) {
            const int kof = kk * 32 + fk;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const __bf16 *ap = As + (32 * mh + 16 * i + fr) * LDSK + kof;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    accg[i][j] = mfma_bf16(ap, Bs + (32 * nh + 16 * j + fr) * LDSK + kof, accg[i][j]);
                    accu[i][j] = mfma_bf16(ap, Bs + (BNH + 32 * nh + 16 * j + fr) * LDSK + kof, accu[i][j]);
                }
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = 32 * mh + 16 * i + 4 * (lane >> 4) + r;
                const int n = 32 * nh + 16 * j + fr;
                if (m < tl.nrows)
                    a.hs[(size_t)(tl.row0 + m) * I + n0 + n] = (__bf16)(silu(accg[i][j][r]) * accu[i][j][r]);
            }
}

// ---------------------------------------------------------------- down
template <int H, int I>
__global__ __launch_bounds__(256) void k_pf_down(PrefillArgs a) {
    constexpr int BM = PF_BM, BN = 64, BK = PF_BK, LDSK = PF_LDSK;
    constexpr int ROWB = (I / QK) * SB_BYTES;
    constexpr int NSTEP = I / BK;
    static_assert(I % BK == 0 && H % BN == 0, "tile shape");
    __shared__ __attribute__((aligned(16))) __bf16 As[BM * LDSK];
    __shared__ __attribute__((aligned(16))) __bf16 Bs[BN * LDSK];

    const Tile tl = a.tiles[blockIdx.x];
    if (tl.expert < 0) return;
    const int e = tl.expert;
    const int n0 = blockIdx.y * BN;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;

    const int am = tid >> 2, aq = tid & 3;
    const bool arow = am < tl.nrows;
    const __bf16 *asrc = a.hs + (size_t)(tl.row0 + (arow ? am : 0)) * I + 32 * aq;
    const int br = tid >> 2, bj = tid & 3;
    const uint8_t *brow = expert_w(a.L.w2, a.L.s2, a.L.sw2, e, a.E) + (size_t)(n0 + br) * ROWB;

    u32x4 ra[4];
    u32x2 rh;
    u32x4 rq;
    auto gload = [&](int step) {
        const int k0 = step * BK;
#pragma unroll
        for (int i = 0; i < 4; ++i) ra[i] = arow ? ldg<u32x4>(asrc + k0 + 8 * i) : u32x4{0, 0, 0, 0};
        const int g = k0 / 32 + bj;
        const uint8_t *sbp = brow + (size_t)(g >> 3) * SB_BYTES;
        rh = ldg<u32x2>(sbp);
        rq = ldg<u32x4>(sbp + 8 + 16 * (g & 7));
    };

    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0, 0, 0, 0};
    const int mh = wv & 1, nh = wv >> 1;
    const int fr = lane & 15, fk = 8 * (lane >> 4);

    gload(0);
    for (int step = 0; step < NSTEP; ++step) {
        {
            u32x4 *ad = reinterpret_cast<u32x4 *>(As + am * LDSK + 32 * aq);
#pragma unroll
            for (int i = 0; i < 4; ++i) ad[i] = ra[i];
            const int g = (step * BK) / 32 + bj;
            dequant_sub_bf16(rq, sub_scale(rh, g & 7), Bs + br * LDSK + 32 * bj);
        }
        __syncthreads();
        if (step + 1 < NSTEP) gload(step + 1);
#pragma unroll
        for (int kk = 0; kk < BK / 32; ++kk) {
            const int kof = kk * 32 + fk;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const __bf16 *ap = As + (32 * mh + 16 * i + fr) * LDSK + kof;
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = mfma_bf16(ap, Bs + (32 * nh + 16 * j + fr) * LDSK + kof, acc[i][j]);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = 32 * mh + 16 * i + 4 * (lane >> 4) + r;
            if (m >= tl.nrows) continue;
            const float sc = a.c * a.sorted_w[tl.row0 + m];
            float *prow = a.part + (size_t)(tl.row0 + m) * H + n0;
#pragma unroll
            for (int j = 0; j < 2; ++j) prow[32 * nh + 16 * j + fr] = sc * acc[i][j][r];
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
static hipError_t launch_prefill_t(const PrefillArgs &a, hipStream_t st, KernelTimer *T) {
    {
        TimedLaunch tl(T, MOE_K_PREFILL_PREP, st);
        hipLaunchKernelGGL((k_pf_prep<H>), dim3(a.M), dim3(256), 0, st, a);
    }
    {
        TimedLaunch tl(T, MOE_K_PREFILL_GATE_UP, st);
        hipLaunchKernelGGL((k_pf_gate_up<H, I>), dim3(a.tile_max, I / 64), dim3(256), 0, st, a);
    }
    {
        TimedLaunch tl(T, MOE_K_PREFILL_DOWN, st);
        hipLaunchKernelGGL((k_pf_down<H, I>), dim3(a.tile_max, H / 64), dim3(256), 0, st, a);
    }
    {
        TimedLaunch tl(T, MOE_K_PREFILL_COMBINE, st);
        hipLaunchKernelGGL((k_pf_combine<H>), dim3(a.M), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

hipError_t launch_prefill(int H, int I, const PrefillArgs &a, hipStream_t st, KernelTimer *T) {
    if (H == 2048 && I == 512) return launch_prefill_t<2048, 512>(a, st, T);
    if (H == 512 && I == 256) return launch_prefill_t<512, 256>(a, st, T);
    return hipErrorInvalidValue;
}

} // namespace moe
