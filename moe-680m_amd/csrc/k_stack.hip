// k_stack.hip -- decode (M = 1) through a stack of MoE layers in one persistent launch.
//
// Replaces, for one token, the per-layer sequence of the reference's forward_single
// restricted to the MoE path (src/inference.rs:296-301): RouterTopk dispatch + blocking
// submit + do_route readback + record_and_submit_moe (18 dispatches, 18 barriers and a
// second blocking submit per layer).  Per layer l:
//     (ids, w) = top8(softmax(logits_l));  x <- x + c * sum_s w_s W2_s(silu(W1_s xin) * W3_s xin)
// with xin = RMSNorm(x) when asked.
//
// Why one persistent kernel: a layer is only 15 MB of IQ4_XS weights (1.9 us at 8 TB/s),
// and its two data dependencies (x -> h -> next x) are global.  On MI355X a kernel boundary
// costs ~1.6 us and an atomic grid barrier over 256 workgroups ~8 us, so both the HBM
// latency and the synchronisation must come off the critical path:
//   - the routing of layer l+2 is computed during layer l by a dedicated router wave, and
//     every wave then issues the loads of its share of layer l+2's weights into registers
//     (two register slots, even/odd layers), so weights stream from HBM two layers ahead;
//   - x_l and h_l are exchanged through per-layer buffers cleared to zero before the
//     launch; producers store each f32 with its mantissa LSB forced to 1 (<= 1 ulp) using
//     agent-scope stores, consumers poll exactly the words they need with agent-scope loads
//     until every word carries the tag.  No atomics, no fences, no barrier: a phase
//     transition costs one cross-XCD store->load round trip (~1.4 us measured).
// Every wait is bounded: a poll that exceeds its limit raises MOE_DEVFLAG_TIMEOUT and a
// global abort word that makes every other poller stop waiting, so all waves always exit.
// The launch needs all NB workgroups resident at once (one per CU); the host checks this.
//
// Work split (NB workgroups; per workgroup 9 compute waves, 1 router wave and 2 poller
// waves, so that no polling load ever queues behind a weight prefetch in a wave's
// in-order load counter):
//   phase A: the 9*I (W1,W3) row pairs, RPW_A consecutive pairs per compute wave, a lane
//            owning one 32-weight sub-block of the row (as in k_decode_gate_up);
//   phase B: WG w owns output rows [8w, 8w+8); compute wave s takes slot s's W2 rows, the
//            nine contributions are summed in slot order in LDS, the residual added.
#include "moe_internal.hpp"

namespace moe {

constexpr uint32_t STK_SPIN_MAX = 1u << 16;

__device__ __forceinline__ void tag_store(uint32_t *p, float v) {
    __hip_atomic_store((MOE_GLOBAL uint32_t *)p, __builtin_bit_cast(uint32_t, v) | 1u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// LDS index of word k with 4 pad words after every 32 (conflict-free 128-bit reads of a
// lane's 32-float chunk).
__device__ __forceinline__ int padk(int k) { return k + ((k >> 5) << 2); }

// One 16-byte coherent load (four tagged words).  A volatile access compiles to a
// system-scope load (sc0 sc1): it misses the CU's L1 and the L2 returns the line as last
// written by any XCD.
__device__ __forceinline__ u32x4 qload(const u32x4 *p) { return *(const volatile MOE_GLOBAL u32x4 *)p; }
__device__ __forceinline__ uint32_t qtag(u32x4 v) { return v[0] & v[1] & v[2] & v[3] & 1u; }

// This thread's share of n tagged words -- 16-byte quads tid, tid+nt, ... (at most MAXQ) --
// polled into LDS.  All loads of a round are in flight together; a round ends with one
// wave-wide test, and only the quads still untagged are reloaded.  The loop is kept short
// on purpose: the time from a producer's store to the end of the wait is dominated by how
// often each word is re-read.  Every wait is bounded (see the file comment).
template <int MAXQ>
__device__ __forceinline__ void poll_quads(const uint32_t *__restrict__ src, float *dst, int n, int tid, int nt,
                                           uint32_t *flags, volatile __attribute__((address_space(3))) int *s_abort) {
    const u32x4 *src4 = reinterpret_cast<const u32x4 *>(src);
    const int nq = n / 4;
    u32x4 v[MAXQ];
#pragma unroll
    for (int j = 0; j < MAXQ; ++j) v[j] = (tid + j * nt < nq) ? qload(src4 + tid + j * nt) : u32x4{1u, 1u, 1u, 1u};
    uint32_t spins = 0;
    while (true) {
        uint32_t t = 1u;
#pragma unroll
        for (int j = 0; j < MAXQ; ++j) t &= qtag(v[j]);
        if (__all(t)) break;
        if ((++spins & 31u) == 0) {
            if (*s_abort) break;
            if (__hip_atomic_load((const MOE_GLOBAL uint32_t *)(flags + 1), __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT)) {
                *s_abort = 1;
                break;
            }
            if (spins >= STK_SPIN_MAX) {
                set_flag(flags, MOE_DEVFLAG_TIMEOUT);
                set_flag(flags + 1, 1u);
                *s_abort = 1;
                break;
            }
        }
#pragma unroll
        for (int j = 0; j < MAXQ; ++j)
            if (!qtag(v[j])) v[j] = qload(src4 + tid + j * nt);
    }
#pragma unroll
    for (int j = 0; j < MAXQ; ++j) {
        const int q = tid + j * nt;
        if (q < nq) *reinterpret_cast<u32x4 *>(dst + padk(4 * q)) = v[j];
    }
}

template <int H, int I>
__global__ __launch_bounds__(64 * STK_WAVES) void k_decode_stack(StackArgs a) {
    constexpr int NB = H / 8;                // workgroups; each owns 8 output rows
    constexpr int LPR1 = (H / QK) * 8;       // lanes per W1/W3 row
    constexpr int RPS1 = 64 / LPR1;          // rows per wave step (phase A)
    constexpr int ROWB1 = (H / QK) * SB_BYTES;
    constexpr int RPW_A = I / NB;            // row pairs per compute wave
    static_assert(RPW_A % RPS1 == 0 && RPW_A >= RPS1, "phase A split");
    constexpr int STA = RPW_A / RPS1;        // phase A steps
    constexpr int LPR2 = (I / QK) * 8;       // lanes per W2 row
    constexpr int RPS2 = 64 / LPR2;          // W2 rows per wave step
    constexpr int ROWB2 = (I / QK) * SB_BYTES;
    static_assert(8 % RPS2 == 0, "phase B split");
    constexpr int STB = 8 / RPS2;            // phase B steps
    constexpr int XPAD = H + (H / 32) * 4;
    constexpr int HPAD = I + (I / 32) * 4;
    constexpr int NPOLL = 64 * (STK_WAVES - SLOTS - 1);     // polling threads (poller waves)
    constexpr int XP = (H / 4 + NPOLL - 1) / NPOLL;         // quads per poller: x
    constexpr int HP = (SLOTS * I / 4 + NPOLL - 1) / NPOLL; // quads per poller: h

    __shared__ __attribute__((aligned(16))) float xs[XPAD];
    __shared__ __attribute__((aligned(16))) float hs[SLOTS * HPAD];
    __shared__ float part[SLOTS][8];
    __shared__ int rt_id[3][SLOTS];
    __shared__ float rt_w[3][SLOTS];
    __shared__ const uint8_t *rt_p[3][SLOTS][3]; // per slot: W1, W3, W2 of the routed expert
    __shared__ int s_abort;

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wg = blockIdx.x;
    const int n = a.n_layers;
    if (tid == 0) s_abort = 0;
    volatile __attribute__((address_space(3))) int *abort_lds =
        (volatile __attribute__((address_space(3))) int *)&s_abort;

    // phase A assignment of compute wave wv
    const int rp0 = (wg * SLOTS + wv) * RPW_A;       // first row pair (valid for wv < 9)
    const int sA = rp0 / I, nA0 = rp0 % I;
    const int g1 = lane % LPR1, rr1 = lane / LPR1, sb1 = g1 >> 3, ib1 = g1 & 7;
    // phase B assignment: slot wv, rows 8*wg + step*RPS2 + rr2
    const int g2 = lane % LPR2, rr2 = lane / LPR2, sb2 = g2 >> 3, ib2 = g2 & 7;

    // Each role runs its own loop; all three execute the same sequence of LDS barriers:
    //   prologue: B0 ; per layer: B1 (x_l in LDS), B2 (h_l in LDS), B3 (partials in LDS),
    //   B4 (x_{l+1} published).  Separate loops keep each role's registers to itself.
    if (wv == SLOTS) {
        // ---------------- router wave: routing two layers ahead into the LDS ring
        auto route = [&](int li) __attribute__((always_inline)) {
            int sel[TOPK];
            float ws[TOPK];
            route_wave<4>(a.logits + (size_t)li * a.E, a.E, a.renorm, lane, sel, ws);
            // the layer table entry is read here, two layers ahead, so that the compute
            // waves' weight prefetches never wait on it
            const LayerPtrs L = load_layer(a.layers + a.layer0 + li);
            if (lane < SLOTS) {
                int id = a.E;
                float wt = 1.0f;
#pragma unroll
                for (int r = 0; r < TOPK; ++r)
                    if (lane == r) { id = sel[r]; wt = ws[r]; }
                rt_id[li % 3][lane] = id;
                rt_w[li % 3][lane] = wt;
                rt_p[li % 3][lane][0] = expert_w(L.w1, L.s1, L.sw1, id, a.E);
                rt_p[li % 3][lane][1] = expert_w(L.w3, L.s3, L.sw3, id, a.E);
                rt_p[li % 3][lane][2] = expert_w(L.w2, L.s2, L.sw2, id, a.E);
            }
            if (wg == 0 && a.ids_out && lane < SLOTS) {
                int id = a.E;
                float wt = 1.0f;
#pragma unroll
                for (int r = 0; r < TOPK; ++r)
                    if (lane == r) { id = sel[r]; wt = ws[r]; }
                *(MOE_GLOBAL uint16_t *)(a.ids_out + (size_t)li * SLOTS + lane) = (uint16_t)id;
                *(MOE_GLOBAL float *)(a.w_out + (size_t)li * SLOTS + lane) = wt;
            }
        };
        route(0);
        if (n > 1) route(1);
        lds_barrier(); // B0
        for (int li = 0; li < n; ++li) {
            if (li + 2 < n) route(li + 2); // ring slot (li+2)%3 was last read before B4 of li-1
            lds_barrier();                 // B1
            lds_barrier();                 // B2
            lds_barrier();                 // B3
            lds_barrier();                 // B4
        }
        return;
    }

    if (wv > SLOTS) {
        // ---------------- poller waves: x_l and h_l into LDS
        const int ptid = tid - 64 * (SLOTS + 1);
        lds_barrier(); // B0
        for (int li = 0; li < n; ++li) {
            if (li == 0) {
                for (int k = ptid; k < H / 4; k += NPOLL) {
                    f32x4 v = ldg<f32x4>(a.x + 4 * k);
                    *reinterpret_cast<f32x4 *>(xs + padk(4 * k)) = v;
                }
            } else {
                poll_quads<XP>(a.xt + (size_t)li * H, xs, H, ptid, NPOLL, a.flags, abort_lds);
            }
            lds_barrier(); // B1
            poll_quads<HP>(a.ht + (size_t)li * SLOTS * I, hs, SLOTS * I, ptid, NPOLL, a.flags, abort_lds);
            lds_barrier(); // B2
            lds_barrier(); // B3
            lds_barrier(); // B4
        }
        return;
    }

    // ---------------- compute waves (wv = 0..8)
    u32x4 aq1[2][STA], aq3[2][STA], bq[2][STB];
    u32x2 ah1[2][STA], ah3[2][STA], bh[2][STB];

    // Loads of local layer li's phase-A (W1, W3) and phase-B (W2) weights for this wave into
    // register slot SL.  Phase-A weights of layer li+2 are requested as soon as phase A of
    // layer li has consumed its slot, phase-B weights after phase B, so the two bursts
    // land in different exchange waits.
    auto prefetch_a = [&](auto SLc, int li) __attribute__((always_inline)) {
        constexpr int SL = decltype(SLc)::value;
        const uint8_t *W1 = rt_p[li % 3][sA][0];
        const uint8_t *W3 = rt_p[li % 3][sA][1];
#pragma unroll
        for (int st = 0; st < STA; ++st) {
            const size_t off = (size_t)(nA0 + st * RPS1 + rr1) * ROWB1 + (size_t)sb1 * SB_BYTES;
            ah1[SL][st] = ldg<u32x2>(W1 + off);
            aq1[SL][st] = ldg<u32x4>(W1 + off + 8 + 16 * ib1);
            ah3[SL][st] = ldg<u32x2>(W3 + off);
            aq3[SL][st] = ldg<u32x4>(W3 + off + 8 + 16 * ib1);
        }
    };
    auto prefetch_b = [&](auto SLc, int li) __attribute__((always_inline)) {
        constexpr int SL = decltype(SLc)::value;
        const uint8_t *W2 = rt_p[li % 3][wv][2];
#pragma unroll
        for (int st = 0; st < STB; ++st) {
            const size_t off = (size_t)(8 * wg + st * RPS2 + rr2) * ROWB2 + (size_t)sb2 * SB_BYTES;
            bh[SL][st] = ldg<u32x2>(W2 + off);
            bq[SL][st] = ldg<u32x4>(W2 + off + 8 + 16 * ib2);
        }
    };

    lds_barrier(); // B0: routing of layers 0 and 1 is in LDS
    prefetch_a(std::integral_constant<int, 0>{}, 0);
    prefetch_b(std::integral_constant<int, 0>{}, 0);
    if (n > 1) {
        prefetch_a(std::integral_constant<int, 1>{}, 1);
        prefetch_b(std::integral_constant<int, 1>{}, 1);
    }

    auto layer = [&](auto SLc, int li) __attribute__((always_inline)) {
        constexpr int SL = decltype(SLc)::value;
        lds_barrier(); // B1: x_l in LDS
        // phase A: h = silu(W1 xin) * (W3 xin) for this wave's row pairs
        {
            float xv[32];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                f32x4 q = *reinterpret_cast<const f32x4 *>(xs + padk(32 * g1) + 4 * i);
                xv[4 * i + 0] = q[0];
                xv[4 * i + 1] = q[1];
                xv[4 * i + 2] = q[2];
                xv[4 * i + 3] = q[3];
            }
            if (a.rmsnorm) {
                float ss = 0.f;
#pragma unroll
                for (int i = 0; i < 32; ++i) ss = __builtin_fmaf(xv[i], xv[i], ss);
                ss = lanes_total<LPR1>(ss);
                const float inv = 1.0f / sqrtf(ss * (1.0f / (float)H) + 1e-6f);
#pragma unroll
                for (int i = 0; i < 32; ++i) xv[i] *= inv;
            }
            float xsum = 0.f;
#pragma unroll
            for (int i = 0; i < 32; ++i) xsum += xv[i];
            uint32_t *hdst = a.ht + ((size_t)li * SLOTS + sA) * I;
#pragma unroll
            for (int st = 0; st < STA; ++st) {
                float g = sub_scale(ah1[SL][st], ib1) * subblock_dot(aq1[SL][st], xv, xsum);
                float u = sub_scale(ah3[SL][st], ib1) * subblock_dot(aq3[SL][st], xv, xsum);
                g = lanes_total<LPR1>(g);
                u = lanes_total<LPR1>(u);
                if (g1 == 0) tag_store(hdst + nA0 + st * RPS1 + rr1, silu(g) * u);
            }
        }
        if (li + 2 < n) prefetch_a(SLc, li + 2);
        lds_barrier(); // B2: h_l in LDS
        // phase B: slot wv's W2 rows against h_l
        {
            float hv[32];
            const float *hsrc = hs + wv * HPAD + padk(32 * g2);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                f32x4 q = *reinterpret_cast<const f32x4 *>(hsrc + 4 * i);
                hv[4 * i + 0] = q[0];
                hv[4 * i + 1] = q[1];
                hv[4 * i + 2] = q[2];
                hv[4 * i + 3] = q[3];
            }
            float hsum = 0.f;
#pragma unroll
            for (int i = 0; i < 32; ++i) hsum += hv[i];
            const float wt = a.c * rt_w[li % 3][wv];
#pragma unroll
            for (int st = 0; st < STB; ++st) {
                float d = sub_scale(bh[SL][st], ib2) * subblock_dot(bq[SL][st], hv, hsum);
                d = group_sum<LPR2>(d);
                if (g2 == 0) part[wv][st * RPS2 + rr2] = wt * d;
            }
        }
        // this slot's registers are free: bring in layer li+2 (its routing arrived by B1)
        if (li + 2 < n) prefetch_b(SLc, li + 2);
        lds_barrier(); // B3: partials in LDS
        // combine in slot order + residual; publish x_{l+1}
        if (tid < 8) {
            const int row = 8 * wg + tid;
            float v = xs[padk(row)];
#pragma unroll
            for (int s = 0; s < SLOTS; ++s) v += part[s][tid];
            if (li + 1 < n) tag_store(a.xt + (size_t)(li + 1) * H + row, v);
            else *(MOE_GLOBAL float *)(a.y + row) = v;
        }
        lds_barrier(); // B4
    };

    for (int li = 0; li < n; li += 2) {
        layer(std::integral_constant<int, 0>{}, li);
        if (li + 1 < n) layer(std::integral_constant<int, 1>{}, li + 1);
    }
}

// Clears the tagged exchange buffers and the abort word before a stack launch (a kernel,
// not hipMemsetAsync, so the sequence can be captured into a graph).
__global__ void k_zero_words(uint32_t *__restrict__ p, uint64_t n, uint32_t *flags) {
    if (blockIdx.x == 0 && threadIdx.x == 0) flags[1] = 0u;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

template <int H, int I>
static hipError_t launch_stack_t(const StackArgs &a, hipStream_t st, KernelTimer *T) {
    const uint64_t words = (uint64_t)(a.n_layers + 1) * H + (uint64_t)a.n_layers * SLOTS * I;
    hipLaunchKernelGGL(k_zero_words, dim3(256), dim3(256), 0, st, a.xt, words, a.flags);
    {
        TimedLaunch tl(T, MOE_K_DECODE_STACK, st);
        hipLaunchKernelGGL((k_decode_stack<H, I>), dim3(H / 8), dim3(64 * STK_WAVES), 0, st, a);
    }
    return hipGetLastError();
}

int stack_blocks(int H) { return H / 8; }

hipError_t stack_occupancy(int H, int I, int *blocks_per_cu) {
    if (H == 2048 && I == 512)
        return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, k_decode_stack<2048, 512>,
                                                            64 * STK_WAVES, 0);
    if (H == 512 && I == 256)
        return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, k_decode_stack<512, 256>,
                                                            64 * STK_WAVES, 0);
    return hipErrorInvalidValue;
}

hipError_t launch_stack(int H, int I, const StackArgs &a, hipStream_t st, KernelTimer *T) {
    if (H == 2048 && I == 512) return launch_stack_t<2048, 512>(a, st, T);
    if (H == 512 && I == 256) return launch_stack_t<512, 256>(a, st, T);
    return hipErrorInvalidValue;
}

} // namespace moe
