// k_decode.hip -- decode path (M <= 8): IQ4_XS-dequant GEMV kernels, f32 arithmetic.
//
// Replaces the reference's decode dispatches (src/inference.rs:733-762): per expert a
// w1_w3_fused_m1 GEMV and a w2_scatter_m1 GEMV (shaders/w1_w3_fused_m1.comp,
// shaders/w2_scatter_m1.comp), 18 dispatches and 18 barriers per layer, with SiLU fused
// into the down projection and the combine done as an f16 read-modify-write of the
// hidden state.  Here one layer is two launches:
//   gate_up: every (token, slot, W1/W3 row pair) of the selected experts, SiLU*up fused,
//            RMSNorm of the input fused (each wave holds the whole activation row);
//   down:    one workgroup per 16 or 32 output rows with one wave per slot, the 9 weighted
//            contributions summed in slot order in LDS (deterministic, no atomics) and
//            the residual added in the same store.
// Lane mapping: a lane owns one 32-weight sub-block of a row (8-byte header load +
// 16-byte qs load), so a 2048-wide W1 row is exactly one wave and the lane's 32
// activations stay in registers for every row it visits.
#include "moe_internal.hpp"

namespace moe {

template <int H, int I, int RP>
__global__ __launch_bounds__(256) void k_decode_gate_up(DecodeArgs a) {
    constexpr int SBR = H / QK;     // super-blocks per W1/W3 row
    constexpr int LPR = SBR * 8;    // lanes per row
    static_assert(LPR <= 64 && 64 % LPR == 0, "row must tile a wave");
    constexpr int RPS = 64 / LPR;   // rows per wave step
    constexpr int ROWB = SBR * SB_BYTES;
    constexpr int RPW = RP * RPS;   // rows per wave
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int item = blockIdx.y;
    const int t0 = item / SLOTS;
    const int gsb = lane % LPR, rr = lane / LPR;
    const int sb = gsb >> 3, ib = gsb & 7;
    const int nbase = (blockIdx.x * 4 + wv) * RPW;

    // The activation row does not depend on routing: its loads go out first, then the
    // expert id and, right behind it, the expert's rows.
    float xv[32];
    load32(a.x + (size_t)t0 * H + 32 * gsb, xv);
    const int e = a.ids[item];
    if (e > a.E) {
        if (threadIdx.x == 0 && blockIdx.x == 0) set_flag(a.flags, MOE_DEVFLAG_BAD_ID);
        return;
    }
    const uint8_t *W1 = expert_w(a.L.w1, a.L.s1, a.L.sw1, e, a.E);
    const uint8_t *W3 = expert_w(a.L.w3, a.L.s3, a.L.sw3, e, a.E);
    u32x4 q1[RP], q3[RP];
    u32x2 h1[RP], h3[RP];
#pragma unroll
    for (int r = 0; r < RP; ++r) {
        const size_t off = (size_t)(nbase + r * RPS + rr) * ROWB + (size_t)sb * SB_BYTES;
        h1[r] = ldg<u32x2>(W1 + off);
        q1[r] = ldg<u32x4>(W1 + off + 8 + 16 * ib);
        h3[r] = ldg<u32x2>(W3 + off);
        q3[r] = ldg<u32x4>(W3 + off + 8 + 16 * ib);
    }
    // Every (token, slot) item runs on its own, also when several tokens name the same
    // expert: the repeated row reads are L2 hits, and one item serving all later tokens
    // serialised their work (at M = 8 the shared expert's items did eight tokens each:
    // 42 against 26 us for this kernel).
    auto run = [&](float(&xr)[32], int p) {
        if (a.rmsnorm) {
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < 32; ++i) ss = __builtin_fmaf(xr[i], xr[i], ss);
            ss = lanes_total<LPR>(ss);
            const float inv = 1.0f / sqrtf(ss * (1.0f / (float)H) + 1e-6f);
#pragma unroll
            for (int i = 0; i < 32; ++i) xr[i] *= inv;
        }
        float xs = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) xs += xr[i];
#pragma unroll
        for (int r = 0; r < RP; ++r) {
            float g = sub_scale(h1[r], ib) * subblock_dot(q1[r], xr, xs);
            float u = sub_scale(h3[r], ib) * subblock_dot(q3[r], xr, xs);
            g = lanes_total<LPR>(g);
            u = lanes_total<LPR>(u);
            if (gsb == 0) a.hbuf[(size_t)p * I + nbase + r * RPS + rr] = silu(g) * u;
        }
    };
    run(xv, item);
}

template <int H, int I, int STEPS>
__global__ __launch_bounds__(64 * SLOTS) void k_decode_down(DecodeArgs a) {
    constexpr int SBR = I / QK;
    constexpr int LPR = SBR * 8;
    static_assert(LPR <= 64 && 64 % LPR == 0, "row must tile a wave");
    constexpr int RPS = 64 / LPR;
    constexpr int ROWB = SBR * SB_BYTES;
    constexpr int RPW = RPS * STEPS; // output rows per workgroup
    __shared__ float part[SLOTS][RPW];
    const int lane = threadIdx.x & 63, s = threadIdx.x >> 6;
    const int t = blockIdx.y;
    const int n0 = blockIdx.x * RPW;
    const int gsb = lane % LPR, rr = lane / LPR;
    const int sb = gsb >> 3, ib = gsb & 7;
    const int p = t * SLOTS + s;
    // h and the slot weight do not depend on the expert id: load them first.
    float hv[32];
    load32(a.hbuf + (size_t)p * I + 32 * gsb, hv);
    const float wslot = a.w[p];
    const int e = a.ids[p];
    float v[STEPS];
#pragma unroll
    for (int st = 0; st < STEPS; ++st) v[st] = 0.f;
    if (e <= a.E) {
        const uint8_t *W2 = expert_w(a.L.w2, a.L.s2, a.L.sw2, e, a.E);
        u32x4 q[STEPS];
        u32x2 hd[STEPS];
#pragma unroll
        for (int st = 0; st < STEPS; ++st) {
            const size_t off = (size_t)(n0 + st * RPS + rr) * ROWB + (size_t)sb * SB_BYTES;
            hd[st] = ldg<u32x2>(W2 + off);
            q[st] = ldg<u32x4>(W2 + off + 8 + 16 * ib);
        }
        float hs = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) hs += hv[i];
        const float wt = a.c * wslot;
#pragma unroll
        for (int st = 0; st < STEPS; ++st) {
            float d = sub_scale(hd[st], ib) * subblock_dot(q[st], hv, hs);
            d = group_sum<LPR>(d);
            v[st] = wt * d;
        }
    } else if (lane == 0 && blockIdx.x == 0) {
        set_flag(a.flags, MOE_DEVFLAG_BAD_ID);
    }
    if (gsb == 0) {
#pragma unroll
        for (int st = 0; st < STEPS; ++st) part[s][st * RPS + rr] = v[st];
    }
    __syncthreads();
    if (threadIdx.x < RPW) {
        const int r = threadIdx.x;
        float sum = 0.f;
#pragma unroll
        for (int q = 0; q < SLOTS; ++q) sum += part[q][r];
        float *yp = a.y + (size_t)t * H + n0 + r;
        *yp = (a.accumulate ? *yp : 0.f) + sum;
    }
}

template <int H, int I>
static hipError_t launch_decode_t(const DecodeArgs &a, hipStream_t st, KernelTimer *T) {
    constexpr int RP = 4;
    constexpr int LPR1 = (H / QK) * 8;
    constexpr int RPW1 = RP * (64 / LPR1);
    static_assert(I % (4 * RPW1) == 0, "gate_up grid");
    dim3 g1(I / (4 * RPW1), a.M * SLOTS);
    {
        TimedLaunch tl(T, MOE_K_DECODE_GATE_UP, st);
        hipLaunchKernelGGL((k_decode_gate_up<H, I, RP>), g1, dim3(256), 0, st, a);
    }
    // down: 4 row steps per wave up to 4 tokens, 8 beyond (more rows in flight per wave once
    // there are enough workgroups; measured at M = 2, 4, 8)
    constexpr int LPR2 = (I / QK) * 8;
    constexpr int RPW4 = (64 / LPR2) * 4, RPW8 = (64 / LPR2) * 8;
    static_assert(H % RPW8 == 0, "down grid");
    {
        TimedLaunch tl(T, MOE_K_DECODE_DOWN, st);
        if (a.M <= 4)
            hipLaunchKernelGGL((k_decode_down<H, I, 4>), dim3(H / RPW4, a.M), dim3(64 * SLOTS), 0, st, a);
        else
            hipLaunchKernelGGL((k_decode_down<H, I, 8>), dim3(H / RPW8, a.M), dim3(64 * SLOTS), 0, st, a);
    }
    return hipGetLastError();
}

hipError_t launch_decode(int H, int I, const DecodeArgs &a, hipStream_t st, KernelTimer *T) {
    if (H == 2048 && I == 512) return launch_decode_t<2048, 512>(a, st, T);
    if (H == 512 && I == 256) return launch_decode_t<512, 256>(a, st, T);
    return hipErrorInvalidValue;
}

} // namespace moe
