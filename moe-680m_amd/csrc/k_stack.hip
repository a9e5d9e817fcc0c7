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
//   - the routing is computed inside the launch ahead of use (the logits are inputs):
//     layers 0 and 1 by the compute waves at the start (four waves per layer), layer l+3 by
//     the router wave while the pollers end layer l, into a ring of three slots of expert
//     pointers; every compute wave keeps its weights in flight in registers: layer
//     l+1's phase-A weights are requested when phase A of l is done, layer l's phase-B
//     weights when phase A of l starts (so no weight stream competes with the
//     latency-bound cross-XCD exchange at the end of a layer).  The weights are read from
//     the split copy of each layer (dense qs, then compact headers; k_repack_split) with one
//     header load per wave and layer, and their codebook lookups are done in the waits --
//     layer l+1's phase-A weights after B3 of l, layer l's phase-B weights after its
//     phase A -- so the phases themselves run only the dot products;
//   - activations move between workgroups through per-layer buffers that start zeroed;
//     producers store each f32 with its mantissa LSB forced to 1 (<= 1 ulp), consumers poll
//     exactly the words they need until every word carries the tag.  No atomics, no
//     fences, no grid barrier.  There are two sets of these buffers: a launch uses set
//     (epoch & 1), clears what the previous launch wrote into the other set (its router
//     waves, spread over the layers), and its last XCD-0 reducer to leave advances the
//     epoch -- so no clearing launch precedes the stack, and consecutive launches (graph
//     replays included) alternate sets.
//
// Work split, mapped onto the eight XCDs (each with its own L2).  Workgroup (k, j) runs on
// XCD k (read from the hardware register, so the roles follow where the dispatcher put the
// workgroup) and is the j-th of the NJ = NB/8 workgroups there.  XCD k owns routed slot k
// (the k-th ranked expert) and 1/8 of the shared expert:
//   phase A (x -> h): XCD k computes h for all I rows of slot k and for shared rows
//       [k*I/8, (k+1)*I/8).  Those 9I/8 values are all XCD k's phase B needs, so they are
//       exchanged inside the XCD only: plain stores (the L2 is the XCD's point of
//       coherence) and L1-bypassing agent-scope loads that hit in that L2.
//   phase B (h -> partial): workgroup (k, j) computes, for output rows [64j, 64j+64),
//       c*w_k*W2_k h_k + c*w_sh*W2_sh[:, cols of XCD k] h_sh -- a K-split: the eight
//       XCDs' partials sum to the layer's FFN output.
//   reduce (partial -> x'): workgroup (k, j) gathers the eight partials of its 64 rows
//       across XCDs (the only cross-XCD traffic: 2 KB per workgroup, write-through stores
//       and system-scope loads), adds them to the residual in a fixed order -- every XCD
//       computes bit-identical rows -- and publishes x' inside its XCD, where all NJ
//       workgroups gather the full vector for the next layer.
// One cross-XCD round trip and two L2-local ones per layer, instead of two all-gathers of
// x (8 KB) and h (18 KB) across all 256 workgroups (5.0 us -> 2.6 us measured for the
// exchanges alone).
// Every wait is bounded: a poll that exceeds its limit raises MOE_DEVFLAG_TIMEOUT and a
// global abort word that makes every other poller stop waiting, so all waves always exit.
// The launch needs all NB workgroups resident at once (one per CU) and the dispatcher's
// round-robin placement over the XCDs (workgroups 8j..8j+7 on eight different XCDs); the
// host checks residency, and a placement that broke the second rule would leave some rows
// unproduced and end in the bounded-wait error, never in a silent wrong result.
//
// Per workgroup: 8 compute waves (two per SIMD, identical work: the shared expert's share is
// split by K over all of them), 1 router wave and 2 poller waves, so that no polling load
// ever queues behind a weight prefetch in a wave's in-order load counter.
#include "moe_internal.hpp"

namespace moe {

// Per-phase timeline (a build with -DMOE_STACK_TRACE, libmoe680m_trace.so; moe_stack_trace):
// lane 0 of the named wave stores the 100 MHz device clock (s_memrealtime, one clock for every
// CU) at each event of each layer into trace[(workgroup * n_layers + layer) * STK_TRACE_EV +
// event].  Other builds compile the marks away.
enum StackTraceEvent {
    STK_EV_START = 0,   // router wave: past B0 (layer 0 only)
    STK_EV_X = 1,       // first poller: past B1 (x_l in LDS)
    STK_EV_ROUTED = 2,  // compute wave 0: past BR (activation routing only)
    STK_EV_A = 3,       // compute wave 0: phase A stored
    STK_EV_HPOLL = 4,   // second poller: its h wait satisfied
    STK_EV_H = 5,       // compute wave 0: past B2 (h_l in LDS)
    STK_EV_B = 6,       // compute wave 0: phase B done
    STK_EV_PUB = 7,     // first poller: partial published (past B3)
    STK_EV_GATHER = 8,  // first poller: the eight partials gathered
    STK_EV_XPUB = 9,    // first poller: x_{l+1} published (or y stored, last layer)
    STK_EV_XPOLL = 10,  // second poller: its x_{l+1} wait satisfied
    STK_EV_LGPOLL = 11, // router wave (activation routing only): the XCD's logits gathered
    STK_EV_TOP8 = 12,   // router wave (activation routing only): top-8 computed
    STK_EV_RING = 13,   // router wave (activation routing only): ring slot written
    STK_TRACE_EV_USED = 14
};
static_assert(STK_TRACE_EV_USED <= STK_TRACE_EV, "trace record");
#ifdef MOE_STACK_TRACE
#define STK_MARK(ev, li)                                                                                          \
    do {                                                                                                          \
        if (a.trace && lane == 0)                                                                                 \
            a.trace[((size_t)blockIdx.x * a.n_layers + (size_t)(li)) * STK_TRACE_EV + (ev)] =                    \
                __builtin_amdgcn_s_memrealtime();                                                                 \
    } while (0)
#else
#define STK_MARK(ev, li) \
    do {                 \
    } while (0)
#endif

constexpr int STK_NX = 8;   // XCDs
constexpr uint32_t STK_DONE_ABORT = 1u << 16; // a done-count contribution that vetoes the y store

// XCD-local publish: a plain store, which stays in this XCD's L2.
__device__ __forceinline__ void tag_store_local(uint32_t *p, float v) {
    *(MOE_GLOBAL uint32_t *)p = __builtin_bit_cast(uint32_t, v) | 1u;
}


// LDS index of word k with 4 pad words after every 32 (conflict-free 128-bit reads of a
// lane's 32-float chunk).
__device__ __forceinline__ int padk(int k) { return k + ((k >> 5) << 2); }

// Tag tests: LSB-tagged f32 words, or words that are never zero once published.
struct LsbTag {
    __device__ __forceinline__ uint32_t operator()(u32x4 v) const { return quad_tagged(v); }
};
struct NonzeroTag {
    __device__ __forceinline__ uint32_t operator()(u32x4 v) const {
        return (uint32_t)((v[0] != 0u) & (v[1] != 0u) & (v[2] != 0u) & (v[3] != 0u));
    }
};

// 16-byte loads that miss the CU's L1, as two relaxed 8-byte atomic loads (atomic, so the
// compiler re-issues them on every poll round; relaxed, so it does not wait for each one as
// it does after a volatile load).  Remote: system scope (sc0 sc1) -- the line comes from
// memory as last written through by any XCD.  Local: agent scope (sc1) -- served by this
// XCD's L2, where the plain stores of its workgroups land.
struct RemoteQuads {
    const u32x4 *p;
    __device__ __forceinline__ u32x4 operator()(int q) const { return remote_quad(p + q); }
};
struct LocalQuads {
    const uint64_t *p;
    __device__ __forceinline__ u32x4 operator()(int q) const {
        const MOE_GLOBAL uint64_t *g = (const MOE_GLOBAL uint64_t *)(p + 2 * q);
        const uint64_t lo = __hip_atomic_load(g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint64_t hi = __hip_atomic_load(g + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return u32x4{(uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32)};
    }
};

typedef volatile __attribute__((address_space(3))) int lds_flag;

// Expiry of a bounded wait: the sticky TIMEOUT flag, the launch's abort word (every other
// waiter stops at its next check) and this workgroup's own abort flag.  The abort word holds
// the tag of the launch that raised it (atag, from the launch epoch), so a later launch of a
// different epoch never mistakes an earlier launch's abort for its own.  A recovery restarts
// the epoch at 0, so it clears the abort word too (moe_device_flags, k_flags_take).
__device__ __forceinline__ void stack_abort(uint32_t *flags, uint32_t atag, lds_flag *s_abort) {
    set_flag(flags, MOE_DEVFLAG_TIMEOUT);
    __hip_atomic_store((MOE_GLOBAL uint32_t *)(flags + 1), atag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_abort = 1;
}
__device__ __forceinline__ bool launch_aborted(const uint32_t *flags, uint32_t atag) {
    return __hip_atomic_load((const MOE_GLOBAL uint32_t *)(flags + 1), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT) == atag;
}

// Bounded wait until every quad in v[] is tagged, reloading only the untagged ones.  All
// loads of a round are in flight together; a round ends with one wave-wide test.  After
// spin_max failed rounds (checked every 32 rounds, or every round once past the limit) the
// wait expires; it also gives up when this workgroup or any other has aborted (checked at
// the same points, so a wait whose data is there costs no LDS or flag read).  Returns false
// -- with the abort flag set and the caller's data invalid -- when it gave up.
template <int MAXQ, typename LD, typename TAG = LsbTag>
__device__ __forceinline__ bool poll_until_tagged(u32x4 (&v)[MAXQ], const int (&q)[MAXQ], const LD &ld,
                                                  uint32_t *flags, uint32_t atag, uint32_t spin_max,
                                                  lds_flag *s_abort, TAG tag = TAG{}) {
    uint32_t spins = 0;
    while (true) {
        uint32_t t = 1u;
#pragma unroll
        for (int j = 0; j < MAXQ; ++j) t &= tag(v[j]);
        if (__all(t)) return true;
        ++spins;
        if ((spins & 31u) == 0 || spins > spin_max) {
            if (*s_abort) return false;
            if (launch_aborted(flags, atag)) {
                *s_abort = 1;
                return false;
            }
            if (spins > spin_max) {
                stack_abort(flags, atag, s_abort);
                return false;
            }
        }
#pragma unroll
        for (int j = 0; j < MAXQ; ++j)
            if (!tag(v[j])) v[j] = ld(q[j]);
    }
}

// Bounded wait (same limits as poll_until_tagged) until the XCD-local counter reaches
// target; returns the count seen, or 0 when the wait expired or the launch aborted.
__device__ __forceinline__ uint32_t wait_count(const uint32_t *ctr, uint32_t target, uint32_t *flags,
                                               uint32_t atag, uint32_t spin_max, lds_flag *s_abort) {
    uint32_t spins = 0;
    while (true) {
        const uint32_t c = (uint32_t)__builtin_amdgcn_readfirstlane((int)__hip_atomic_load(
            (const MOE_GLOBAL uint32_t *)ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        if (c >= target) return c;
        ++spins;
        if ((spins & 31u) == 0 || spins > spin_max) {
            if (*s_abort) return 0u;
            if (launch_aborted(flags, atag)) {
                *s_abort = 1;
                return 0u;
            }
            if (spins > spin_max) {
                stack_abort(flags, atag, s_abort);
                return 0u;
            }
        }
    }
}

// Sum over aligned groups of G adjacent lanes (G = 1, 2, 4, 8), result in every lane.
template <int G>
__device__ __forceinline__ float adjacent_sum(float v) {
    if constexpr (G == 1) return v;
    else if constexpr (G == 2) return v + dpp_mov<0xB1>(v);
    else if constexpr (G == 4) {
        v += dpp_mov<0xB1>(v);
        return v + dpp_mov<0x4E>(v);
    } else return group_sum<G>(v);
}

// ---------------------------------------------------------------- int8 activations
// Phase A reads x as the two int8 planes of moe_device.hpp (quant_ratio, subblock_idot).  In
// the exchange, element pair (2w, 2w+1) is one word [xl_2w, xh_2w ^ 0x80, xl_2w+1,
// xh_2w+1 ^ 0x80]: xh is never -128, so byte 1 is never zero and a published word is never
// zero -- the exchange tag is "word != 0" (the zero-cleared buffer), which costs no bit of
// precision.
__device__ __forceinline__ uint32_t pack_pair(float xe, float xo, float r) {
    const float ue = xe * r, uo = xo * r;
    // the clamps also map a non-finite input to a finite byte, so the tag always holds
    const float he = fminf(fmaxf(rintf(ue), -127.0f), 127.0f), ho = fminf(fmaxf(rintf(uo), -127.0f), 127.0f);
    const float le = fminf(fmaxf(rintf((ue - he) * 256.0f), -127.0f), 127.0f);
    const float lo = fminf(fmaxf(rintf((uo - ho) * 256.0f), -127.0f), 127.0f);
    return (((uint32_t)(int)le & 0xFFu) | (((uint32_t)(int)he & 0xFFu) << 8) | (((uint32_t)(int)lo & 0xFFu) << 16) |
            (((uint32_t)(int)ho & 0xFFu) << 24)) ^ 0x80008000u;
}

// Exchange quad q (elements 8q..8q+7, four pair words) into the planes.
__device__ __forceinline__ void store_quad(uint32_t *xq, int q, u32x4 v) {
    uint32_t *c = xq + XQS * (q >> 2) + 2 * (q & 3);
    *reinterpret_cast<u32x2 *>(c) = u32x2{__builtin_amdgcn_perm(v[1], v[0], 0x07050301u) ^ 0x80808080u,
                                          __builtin_amdgcn_perm(v[3], v[2], 0x07050301u) ^ 0x80808080u};
    *reinterpret_cast<u32x2 *>(c + 8) =
        u32x2{__builtin_amdgcn_perm(v[1], v[0], 0x06040200u), __builtin_amdgcn_perm(v[3], v[2], 0x06040200u)};
}

// 16-byte quads of one layer block of an exchange set (stack_layer_words / 4).
template <int H, int I>
__host__ __device__ constexpr uint64_t stack_layer_quads() {
    return (uint64_t)STK_NX * (3 * I + H + H / 2 + H / 32 + H / 64 + STK_LG_WORDS) / 4;
}
static_assert(stack_layer_quads<2048, 512>() * 4 ==
                  (uint64_t)STK_NX * (3 * 512 + 2048 + 1024 + 64 + 32 + STK_LG_WORDS),
              "whole quads per layer block");

// AR (StackArgs::logits null): every layer is routed from its own input.  Per layer, after
// x_l is in LDS (B1), every compute wave takes one router row's dot with it -- row
// (j * NCW + w) * RPS1 + rr1 of the layer's gate matrix (IQ4_XS, f32 or f16, requested
// while the previous layer's x was exchanged), against the same int8 planes phase A reads --
// and publishes the logit inside its XCD; the router wave gathers all E, routes the layer and
// fills its ring slot; one more LDS barrier (BR) hands the routing to the compute waves, which
// only then request that layer's expert weights.  Every XCD computes the same logits from the
// same planes, so all eight agree on the routing.  Logits are LSB-tagged (<= 1 ulp).
template <int H, int I, bool AR>
__global__ __launch_bounds__(64 * STK_WAVES) void k_decode_stack(StackArgs a) {
    constexpr int NX = STK_NX;
    constexpr int NCW = STK_CWAVES;          // compute waves, two per SIMD
    constexpr int NB = H / 8;                // workgroups
    constexpr int NJ = NB / NX;              // workgroups per XCD
    constexpr int ROWS = H / NJ;             // output rows per workgroup
    static_assert(NB % NX == 0 && ROWS == 64 && ROWS == 8 * NCW, "one 64-row block per workgroup");
    constexpr int SRP = I / NB;              // shared-expert row pairs per workgroup
    constexpr int HX = I + I / NX;           // h of one XCD in LDS: routed slot, then shared share
    constexpr int HXG = 3 * I;               // ... in the exchange buffer (see phase A)
    constexpr int CPX = I / (32 * NX);       // shared-expert 32-column chunks per XCD
    static_assert(CPX == 1 || CPX == 2, "shared split");
    // phase A, slot k: SRP row pairs per compute wave, a lane owning one sub-block of a row
    constexpr int LPR1 = (H / QK) * 8;       // lanes per W1/W3 row
    constexpr int RPS1 = 64 / LPR1;          // rows per wave step
    static_assert(SRP % RPS1 == 0 && SRP >= RPS1, "phase A split");
    static_assert(8 * SRP * NJ == I && SRP * NJ == I / NX, "phase A covers slot k and the shared share");
    constexpr int STA = SRP / RPS1;
    // phase A, shared: the workgroup's 2*SRP shared rows, K split over the compute waves,
    // a lane owning half a sub-block (16 weights)
    constexpr int SBW = H / (32 * NCW);      // sub-blocks per wave per row
    constexpr int LPRS = 2 * SBW;            // lanes per shared row
    constexpr int NSA = 2 * SRP * LPRS;      // lanes in use
    static_assert(NSA <= 64 && (LPRS & (LPRS - 1)) == 0, "shared phase A split");
    // phase B: compute wave w owns rows 8w..8w+7 of the workgroup's block: all I columns of
    // W2_k (one sub-block per lane), and the XCD's CPX shared chunks (one qs dword per lane)
    constexpr int LPR2 = (I / QK) * 8;       // lanes per W2 row
    constexpr int RPS2 = 64 / LPR2;
    static_assert(8 % RPS2 == 0, "phase B split");
    constexpr int STB = 8 / RPS2;
    constexpr int LPRB = 4 * CPX;            // lanes per row, shared part
    constexpr int NSB = 8 * LPRB;
    static_assert(NSB <= 64, "shared phase B split");
    constexpr int NCH = H / 32;              // x chunks (= sub-blocks along K)
    constexpr int HPAD = HX + (HX / 32) * 4 + 4;
    constexpr int NPOLL = 64 * (STK_WAVES - NCW - 1);       // polling threads (poller waves)
    static_assert(NPOLL == 128, "two poller waves");
    // x exchange of one (layer, XCD): H/2 pair words, H/32 chunk scales, NJ per-workgroup
    // sums of squares -- XQ quads
    constexpr int XD = H / 8, XS = H / 128, NSS = NJ / 4, XQ = XD + XS + NSS;
    static_assert(NSS >= 2 && 4 * XQ == H / 2 + H / 32 + NJ, "x exchange layout");
    constexpr int XP = (XQ + NPOLL - 1) / NPOLL;            // quads per poller: x
    static_assert(I / NX <= 64 && I / 4 <= 4 * 64 && (I / 4) % 64 == 0, "h gather split");

    __shared__ __attribute__((aligned(16))) uint32_t xq[NCH * XQS]; // x as int8 planes
    __shared__ __attribute__((aligned(16))) float xsc[NCH];         // ... and chunk scales
    __shared__ __attribute__((aligned(16))) float ssq[NSS];         // partial sums of x^2
    __shared__ __attribute__((aligned(16))) float hs[HPAD];
    __shared__ float hsm[I / 32];       // sums of h_k's 32-element chunks
    __shared__ float part[2][ROWS];     // this workgroup's slot-k and shared contributions
    __shared__ __attribute__((aligned(16))) float ps[NX][ROWS]; // the eight XCD partials of its rows
    __shared__ float rt_w[3][2];        // per layer (ring of 3): weight of slot k, shared
    __shared__ const uint8_t *rt_p[3][2][3]; // W1, W3, W2 of the routed expert / shared
    __shared__ int s_abort;
    __shared__ int s_j;
    __shared__ uint32_t s_ep;
    __shared__ __attribute__((aligned(16))) float s_lg[STK_LG_WORDS]; // AR: a layer's logits

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    // HW_REG_XCC_ID (readfirstlane: the compiler then knows the value is wave-uniform)
    const int k = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & (NX - 1));
    const int n = a.n_layers;
    lds_flag *abort_lds = (lds_flag *)&s_abort;
    auto ctl = [&](int w) { return a.ctl + (size_t)w * STK_CTL_STRIDE; };

    // Layer r's routing into ring slot r % 3: the id and weight of slot k (lane s of a routing
    // result holds rank s; lanes 8 and up the shared expert) and the weight pointers; the
    // first workgroup also publishes the layer's ids and weights.
    auto ring_write = [&](int r, int id, float wt, const LayerPtrs &L) __attribute__((always_inline)) {
        const int idk = __builtin_amdgcn_readlane(id, k);
        const float wk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wt), k));
        if (lane < 2) {
            const int e = lane == 0 ? idk : a.E;
            rt_w[r % 3][lane] = lane == 0 ? wk : 1.0f;
            rt_p[r % 3][lane][0] = expert_w(L.w1, L.s1, L.sw1, e, a.E);
            rt_p[r % 3][lane][1] = expert_w(L.w3, L.s3, L.sw3, e, a.E);
            rt_p[r % 3][lane][2] = expert_w(L.w2, L.s2, L.sw2, e, a.E);
        }
        if (blockIdx.x == 0 && a.ids_out && lane < SLOTS) {
            a.ids_out[(size_t)r * SLOTS + lane] = (uint16_t)id;
            a.w_out[(size_t)r * SLOTS + lane] = wt;
        }
    };

    // Start: compute wave 0 routes layer 0 and wave 4 layer 1 (the one-wave top-8, no barrier);
    // the router wave takes this
    // workgroup's rank j among the workgroups that started on XCD k -- a per-XCD ticket, not
    // blockIdx, so no assumption on the dispatch order -- and the launch epoch meanwhile.  An
    // XCD that receives more than NJ workgroups leaves another XCD short: the surplus ones
    // raise the timeout and leave, and the others' bounded waits end the launch with y
    // untouched.
    if (wv < NCW) {
        if constexpr (!AR) {
            const int grp = wv >> 2, r = grp < n ? grp : 0;
            if ((wv & 3) == 0) {
                const LayerPtrs L = load_layer(a.layers + a.layer0 + r);
                float raw[4];
                load_logits<4>(a.logits + (size_t)r * a.E, a.E, lane, raw);
                int id;
                float wt;
                route_values<4>(raw, a.E, a.renorm, lane, id, wt);
                if (grp < n) ring_write(grp, id, wt, L);
            }
        }
    } else {
        // the ticket and the epoch, waited for after the routing (B0 follows)
        const bool tk = wv == NCW && lane == 0;
        uint32_t t = 0u, e0 = 0u;
        if (tk) {
            t = __hip_atomic_fetch_add((MOE_GLOBAL uint32_t *)ctl(k), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            e0 = __hip_atomic_load((const MOE_GLOBAL uint32_t *)ctl(STK_CTL_EPOCH), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
        if (tk) {
            s_j = t < (uint32_t)NJ ? (int)t : -1;
            s_ep = e0;
            s_abort = 0;
        }
    }
    lds_barrier(); // B0: routing of layers 0 and 1, ticket and epoch in LDS
    const int j = s_j;
    const uint32_t ep = s_ep;
    const uint32_t atag = ep | 0x80000000u; // this launch's abort-word value (never 0)
    uint32_t *const xset = a.xs + (size_t)(ep & 1u) * a.set_words;

    // The other exchange set: the previous launch used it; this launch clears the layer blocks
    // it wrote, in n + 1 pieces (one per router-wave window), workgroup b taking an equal,
    // 512-byte aligned share -- by blockIdx, so surplus workgroups do theirs too.
    uint32_t dirty_o = 0u; // layer blocks of the other set to clear (read by the router wave)
    if (wv == NCW)
        dirty_o = min(ldg<uint32_t>(ctl(STK_CTL_DIRTY + (int)((ep & 1u) ^ 1u))), (uint32_t)a.n_max);
    auto clear_other = [&](int piece, int pieces) __attribute__((always_inline)) {
        const uint32_t o = (ep & 1u) ^ 1u;
        const uint64_t Q = (uint64_t)dirty_o * stack_layer_quads<H, I>();
        const uint64_t per = ((Q + NB - 1) / NB + 31) & ~(uint64_t)31;
        const uint64_t q0 = min((uint64_t)blockIdx.x * per, Q), q1 = min(q0 + per, Q);
        const uint64_t b0 = q0 + (q1 - q0) * (uint64_t)piece / pieces, b1 = q0 + (q1 - q0) * (uint64_t)(piece + 1) / pieces;
        u32x4 *dst = reinterpret_cast<u32x4 *>(a.xs + (size_t)o * a.set_words);
        for (uint64_t q = b0 + lane; q < b1; q += 64) *(MOE_GLOBAL u32x4 *)(dst + q) = u32x4{0u, 0u, 0u, 0u};
    };
    if (j < 0) {
        if (wv == NCW) {
            clear_other(0, 1);
            if (lane == 0) stack_abort(a.flags, atag, abort_lds);
        }
        return;
    }

    // exchange buffers of (layer li, XCD k) in this launch's set: one block per layer
    constexpr size_t LW = 4 * stack_layer_quads<H, I>();
    auto hbuf = [&](int li) { return xset + (size_t)li * LW + (size_t)k * HXG; };
    auto pbuf = [&](int li) { return xset + (size_t)li * LW + (size_t)NX * HXG; };
    auto xbuf = [&](int li) { return xset + (size_t)li * LW + (size_t)NX * (HXG + H) + (size_t)k * (4 * XQ); }; // x_{li+1}
    auto lbuf = [&](int li) { // AR: layer li's logits
        return xset + (size_t)li * LW + (size_t)NX * (HXG + H + 4 * XQ) + (size_t)k * STK_LG_WORDS;
    };
    const int E4 = (a.E + 3) & ~3; // AR: logit words published (rows E..E4-1 as dummies)

    if (wv == NCW) {
        if constexpr (AR) {
            // ---------------- router wave (AR): routes layer li from the logits that every
            // workgroup of this XCD published after B1 of li, into ring slot li % 3 before BR;
            // clears the other exchange set in n + 1 pieces, as below
            if (blockIdx.x == 0 && lane == 0)
                __hip_atomic_store((MOE_GLOBAL uint32_t *)ctl(STK_CTL_DIRTY + (int)(ep & 1u)), (uint32_t)n,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            STK_MARK(STK_EV_START, 0);
            clear_other(0, n + 1);
            const int nq = E4 >> 2;
            for (int li = 0; li < n; ++li) {
                const LayerPtrs L = load_layer(a.layers + a.layer0 + li);
                lds_barrier(); // B1: x_li in LDS, its logits being published
                {
                    const LocalQuads ld{reinterpret_cast<const uint64_t *>(lbuf(li))};
                    int q[1] = {lane};
                    u32x4 v[1] = {lane < nq ? ld(lane) : u32x4{1u, 1u, 1u, 1u}};
                    // a wait that gives up leaves the abort flag set: stale logits then still
                    // route to valid expert ids, and nothing computed from them is published
                    (void)poll_until_tagged<1>(v, q, ld, a.flags, atag, a.spin_max, abort_lds);
                    STK_MARK(STK_EV_LGPOLL, li);
                    if (lane < nq) *reinterpret_cast<f32x4 *>(s_lg + 4 * lane) = __builtin_bit_cast(f32x4, v[0]);
                    // lanes read what other lanes of this wave wrote: LDS keeps a wave's
                    // accesses in order, the compiler must too
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                    float raw[4];
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) raw[jj] = s_lg[min(lane + 64 * jj, a.E - 1)];
                    int id;
                    float wt;
                    __builtin_amdgcn_s_setprio(3);
                    route_values<4>(raw, a.E, a.renorm, lane, id, wt);
                    STK_MARK(STK_EV_TOP8, li);
                    __builtin_amdgcn_s_setprio(0);
                    ring_write(li, id, wt, L);
                    STK_MARK(STK_EV_RING, li);
                }
                lds_barrier(); // BR: routing of li in LDS
                lds_barrier(); // B2
                // every workgroup of the XCD published its h of layer 0, so all took their
                // tickets: reset the XCD's counter for the next launch
                if (li == 0 && j == 0 && lane == 0 && !*abort_lds)
                    __hip_atomic_store((MOE_GLOBAL uint32_t *)ctl(k), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                lds_barrier(); // B3
                clear_other(li + 1, n + 1);
            }
            return;
        } else {
            // ---------------- router wave: routes layer r + 3 into ring slot r % 3 while the
            // pollers end layer r (after B3; that slot was last read in phase B of r and is next
            // read at B2 of r + 2), layer 2 right after B0; clears the other exchange set.
            float raw[4];
            LayerPtrs L;
            auto fetch = [&](int r) __attribute__((always_inline)) {
                load_logits<4>(a.logits + (size_t)r * a.E, a.E, lane, raw);
                L = load_layer(a.layers + a.layer0 + r);
            };
            auto route = [&](int r) __attribute__((always_inline)) {
                int id;
                float wt;
                route_values<4>(raw, a.E, a.renorm, lane, id, wt);
                ring_write(r, id, wt, L);
                if (r + 1 < n) fetch(r + 1);
            };
            if (blockIdx.x == 0 && lane == 0)
                __hip_atomic_store((MOE_GLOBAL uint32_t *)ctl(STK_CTL_DIRTY + (int)(ep & 1u)), (uint32_t)n,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (n > 2) fetch(2);
            STK_MARK(STK_EV_START, 0);
            // window 0 follows B0, window li + 1 follows B3 of layer li; window w routes layer w + 2
            for (int wdw = 0; wdw <= n; ++wdw) {
                if (wdw > 0) {
                    lds_barrier();             // B1 of layer wdw - 1
                    lds_barrier();             // B2
                    // every workgroup of the XCD published its h of layer 0 (the wait before B2
                    // succeeded), so all took their tickets: reset the XCD's counter for the next
                    // launch
                    if (wdw == 1 && j == 0 && lane == 0 && !*abort_lds)
                        __hip_atomic_store((MOE_GLOBAL uint32_t *)ctl(k), 0u, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                    lds_barrier();             // B3
                }
                // at the priority of the compute waves' phases: at 0 the routing took issue slots
                // behind the compute waves' lookups and reached B1 late (measured +0.5 us per layer)
                __builtin_amdgcn_s_setprio(3);
                if (wdw + 2 < n) route(wdw + 2);
                __builtin_amdgcn_s_setprio(0);
                clear_other(wdw, n + 1);
            }
            return;
        }
    }

    if (wv > NCW) {
        // ---------------- poller waves: x and h into LDS; the first also reduces
        const int ptid = tid - 64 * (NCW + 1);
        const bool first = wv == NCW + 1;
        bool got = true; // every wait of this wave so far ended with its data
        // x_0 from the input: quad q (8 elements) per thread, a chunk on four adjacent lanes
        {
            float ss = 0.f;
            for (int q = ptid; q < XD; q += NPOLL) {
                const f32x4 x0 = ldg<f32x4>(a.x + 8 * q), x1 = ldg<f32x4>(a.x + 8 * q + 4);
                float am = 0.f;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    am = fmaxf(am, fmaxf(fabsf(x0[e]), fabsf(x1[e])));
                    ss = __builtin_fmaf(x0[e], x0[e], ss);
                    ss = __builtin_fmaf(x1[e], x1[e], ss);
                }
                am = fmaxf(am, dpp_mov<0xB1>(am));
                am = fmaxf(am, dpp_mov<0x4E>(am));
                const float r = quant_ratio(am);
                store_quad(xq, q,
                           u32x4{pack_pair(x0[0], x0[1], r), pack_pair(x0[2], x0[3], r),
                                 pack_pair(x1[0], x1[1], r), pack_pair(x1[2], x1[3], r)});
                if ((q & 3) == 0) xsc[q >> 2] = am * (1.0f / 127.0f);
            }
            ss = wave_sum(ss);
            if (lane == 0) ssq[first ? 0 : 1] = ss;
            if (first && lane >= 2 && lane < NSS) ssq[lane] = 0.f;
        }
        // the reducer's own 64 rows of the residual, kept in f32
        float xres = first ? a.x[ROWS * j + lane] : 0.f;
        for (int li = 0; li < n; ++li) {
            lds_barrier(); // B1: x_li in LDS
            if (first) STK_MARK(STK_EV_X, li);
            if constexpr (AR) lds_barrier(); // BR: the layer's routing in LDS
            // the h exchange: ahead of the compute waves' phase-B lookups (priority 0), level
            // with phase A (priority 1; the older compute waves win the ties)
            __builtin_amdgcn_s_setprio(1);
            {
                // h of the XCD: the first poller wave takes the shared rows (lane t: the 16
                // words of shared row t -- eight waves' partial (g, u) -- combined here), the
                // second the routed slot's I words
                const LocalQuads ld{reinterpret_cast<const uint64_t *>(hbuf(li))};
                int q[4];
                u32x4 v[4];
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const bool ok = first ? lane < I / NX : lane + 64 * m < I / 4;
                    q[m] = first ? I / 4 + 4 * lane + m : lane + 64 * m;
                    v[m] = ok ? ld(q[m]) : u32x4{1u, 1u, 1u, 1u};
                }
                got = poll_until_tagged<4>(v, q, ld, a.flags, atag, a.spin_max, abort_lds) && got;
                if (!first) STK_MARK(STK_EV_HPOLL, li);
                if (first) {
                    if (lane < I / NX) {
                        float g = 0.f, u = 0.f;
#pragma unroll
                        for (int m = 0; m < 4; ++m) {
                            // cast the whole vector: a bit_cast of one element of an
                            // ext_vector lvalue reads element 0 with this compiler
                            const f32x4 f = __builtin_bit_cast(f32x4, v[m]);
                            g += f[0];
                            u += f[1];
                            g += f[2];
                            u += f[3];
                        }
                        hs[padk(I + lane)] = silu_rcp(g) * u;
                    }
                } else {
#pragma unroll
                    for (int m = 0; m < 4; ++m)
                        if (64 * m < I / 4) { // wave-uniform: I/4 is a multiple of 64
                            const f32x4 f = __builtin_bit_cast(f32x4, v[m]);
                            *reinterpret_cast<f32x4 *>(hs + padk(4 * q[m])) = f;
                            // chunk sums of h_k (eight adjacent lanes per chunk) for the biased
                            // codebook correction of phase B
                            const float cs = group_sum<8>((f[0] + f[1]) + (f[2] + f[3]));
                            if ((q[m] & 7) == 0) hsm[q[m] >> 3] = cs;
                        }
                }
            }
            lds_barrier(); // B2: h_li in LDS
            lds_barrier(); // B3: every compute wave past phase B (the contributions in LDS)
            // until B1 the compute waves only decode the next layer's weights, which is off
            // the critical path: let the exchange win every VALU issue slot on its SIMD
            __builtin_amdgcn_s_setprio(2);
            if (first) {
                // this XCD's partial of rows [64j, 64j+64): published by the compute waves, or
                // (routed from the activations) here ...
                uint32_t *pb = pbuf(li);
                if constexpr (AR) {
                    // (the workgroup's abort word read with the contributions: a wait that gave
                    // up in another wave of this workgroup left them invalid)
                    const float pv = part[0][lane] + part[1][lane];
                    const int ab = *abort_lds;
                    if (got && !ab) tag_store(pb + (size_t)k * H + ROWS * j + lane, pv);
                }
                STK_MARK(STK_EV_PUB, li);
                // ... then gather all eight (lane: quad lane&15 of XCDs lane>>4 and (lane>>4)+4) ...
                const RemoteQuads ld{reinterpret_cast<const u32x4 *>(pb + ROWS * j)};
                const int m = lane >> 4, qq = lane & 15;
                int q[2] = {m * (H / 4) + qq, (m + 4) * (H / 4) + qq};
                u32x4 v[2] = {ld(q[0]), ld(q[1])};
                got = poll_until_tagged<2>(v, q, ld, a.flags, atag, a.spin_max, abort_lds) && got;
                STK_MARK(STK_EV_GATHER, li);
                *reinterpret_cast<f32x4 *>(&ps[m][4 * qq]) = __builtin_bit_cast(f32x4, v[0]);
                *reinterpret_cast<f32x4 *>(&ps[m + 4][4 * qq]) = __builtin_bit_cast(f32x4, v[1]);
                // lanes read what other lanes of this wave wrote: LDS keeps a wave's
                // accesses in order, the compiler must too
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                // ... and add them to the residual in XCD order (the same on every XCD)
                const int row = ROWS * j + lane;
                float x1 = xres;
#pragma unroll
                for (int s = 0; s < NX; ++s) x1 += ps[s][lane];
                xres = x1;
                if (li + 1 < n) {
                    // publish x' as int8 planes: lanes 0-31 and 32-63 are chunks 2j, 2j+1
                    uint32_t *xb = xbuf(li);
                    float am = fabsf(x1);
                    am = fmaxf(am, dpp_mov<0xB1>(am));
                    am = fmaxf(am, dpp_mov<0x4E>(am));
                    am = fmaxf(am, dpp_mov<0x141>(am));
                    am = fmaxf(am, dpp_mov<0x140>(am));
                    {
                        const auto sw = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, am),
                                                                         __builtin_bit_cast(uint32_t, am), false, false);
                        const uint32_t s0 = sw[0], s1 = sw[1]; // elements by value (whole-vector rule above)
                        am = fmaxf(__builtin_bit_cast(float, s0), __builtin_bit_cast(float, s1));
                    }
                    const float xo = dpp_mov<0xB1>(x1); // the odd partner of an even lane
                    const float ss = wave_sum(x1 * x1);
                    if (got) {
                        if ((lane & 1) == 0)
                            *(MOE_GLOBAL uint32_t *)(xb + (row >> 1)) = pack_pair(x1, xo, quant_ratio(am));
                        if ((lane & 31) == 0) tag_store_local(xb + H / 2 + (row >> 5), am * (1.0f / 127.0f));
                        if (lane == 0) tag_store_local(xb + H / 2 + H / 32 + j, ss);
                    }
                    STK_MARK(STK_EV_XPUB, li);
                } else if (k == 0) {
                    // y is written by all of XCD 0's reducers or by none.  Nothing computed
                    // from a wait that gave up is ever published (a wave publishes only after
                    // its own waits succeeded and, for data other waves left in LDS, with the
                    // workgroup's abort word clear), so a reducer whose waits all succeeded
                    // holds valid rows.  Each adds to a count in that XCD's L2: 1 when sound,
                    // else STK_DONE_ABORT; all NJ write y only on a count of exactly NJ.  An
                    // expired wait anywhere in the launch -- every later wait on what it would
                    // have published expires too -- thus leaves y, and an x it aliases, as it
                    // was.
                    uint32_t *done = ctl(STK_CTL_DONE);
                    const bool sound = got && !*abort_lds;
                    if (lane == 0)
                        __hip_atomic_fetch_add((MOE_GLOBAL uint32_t *)done, sound ? 1u : STK_DONE_ABORT,
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    const uint32_t c = wait_count(done, (uint32_t)NJ, a.flags, atag, a.spin_max, abort_lds);
                    if (c == (uint32_t)NJ)
                        *(MOE_GLOBAL float *)(a.y + row) = x1;
                    else if (c != 0u && lane == 0)
                        set_flag(a.flags, MOE_DEVFLAG_TIMEOUT); // a count past NJ: not every reducer was sound
                    STK_MARK(STK_EV_XPUB, li);
                    // The last of XCD 0's reducers to leave resets the two counts and advances
                    // the epoch, which switches the next launch to the exchange set this launch
                    // cleared.  By then every workgroup of the launch has started (each of them
                    // published a partial this XCD gathered, or left the gathers waiting) and
                    // read the epoch, and every reducer of XCD 0 has passed its wait on `done`.
                    if (lane == 0) {
                        uint32_t *ex = ctl(STK_CTL_EXIT);
                        const uint32_t t = __hip_atomic_fetch_add((MOE_GLOBAL uint32_t *)ex, 1u, __ATOMIC_RELAXED,
                                                                  __HIP_MEMORY_SCOPE_AGENT);
                        if (t == (uint32_t)NJ - 1u) {
                            __hip_atomic_store((MOE_GLOBAL uint32_t *)done, 0u, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
                            __hip_atomic_store((MOE_GLOBAL uint32_t *)ex, 0u, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
                            __hip_atomic_store((MOE_GLOBAL uint32_t *)ctl(STK_CTL_EPOCH), ep + 1u,
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        }
                    }
                }
            }
            if (li + 1 < n) {
                // x_{li+1} of this XCD into the planes, scales and partial sums of squares
                const LocalQuads ld{reinterpret_cast<const uint64_t *>(xbuf(li))};
                int q[XP];
                u32x4 v[XP];
#pragma unroll
                for (int m = 0; m < XP; ++m) {
                    q[m] = ptid + m * NPOLL;
                    v[m] = q[m] < XQ ? ld(q[m]) : u32x4{1u, 1u, 1u, 1u};
                }
                // pair words are tagged by being nonzero; the scales and sums of squares
                // are LSB-tagged f32 words, which are nonzero too
                got = poll_until_tagged<XP>(v, q, ld, a.flags, atag, a.spin_max, abort_lds, NonzeroTag{}) && got;
                if (!first) STK_MARK(STK_EV_XPOLL, li);
#pragma unroll
                for (int m = 0; m < XP; ++m) {
                    if (q[m] < XD) {
                        store_quad(xq, q[m], v[m]);
                    } else if (q[m] < XD + XS) {
                        *reinterpret_cast<f32x4 *>(xsc + 4 * (q[m] - XD)) = __builtin_bit_cast(f32x4, v[m]);
                    } else if (q[m] < XQ) {
                        const f32x4 f = __builtin_bit_cast(f32x4, v[m]);
                        ssq[q[m] - XD - XS] = (f[0] + f[1]) + (f[2] + f[3]);
                    }
                }
            }
        }
        return;
    }

    // ---------------- compute waves (w = wv = 0..7)
    const int w = wv;
    // phase A, slot k: rows (8j + w)*SRP .. +SRP (also their h index)
    const int rowA = (8 * j + w) * SRP;
    const int g1 = lane % LPR1, rr1 = lane / LPR1, sb1 = g1 >> 3, ib1 = g1 & 7;
    // the lane of each row group that holds the row's total (see row_total)
    constexpr int LPR1_LAST = LPR1 == 64 ? 63 : 0;
    // Weights are read from the split copy of the layer (k_repack_split): per matrix, the
    // 128-byte qs of super-block (row, s) at 128 (row * SBR + s), then the 8-byte headers at
    // HDR + 8 (row * SBR + s).
    constexpr int SBR1 = H / QK, SBR2 = I / QK;
    constexpr uint32_t HDR1 = (uint32_t)I * SBR1 * 128, HDR2 = (uint32_t)H * SBR2 * 128;
    uint32_t offA[STA];
#pragma unroll
    for (int st = 0; st < STA; ++st) offA[st] = (uint32_t)(((rowA + st * RPS1 + rr1) * SBR1 + sb1) * 128 + 16 * ib1);
    // phase A, shared: lane -> row ri (pair ri/2, W1 or W3 by ri&1), sub-block sbg of this
    // wave's K range, half hh.  Lanes past NSA repeat valid addresses; their sums are dropped.
    const int ri = (lane / LPRS) % (2 * SRP), pA = ri >> 1, mA = ri & 1;
    const int sbg = w * SBW + ((lane % LPRS) >> 1), hh = lane & 1;
    const uint32_t offSA = (uint32_t)(((k * (I / NX) + j * SRP + pA) * SBR1 + (sbg >> 3)) * 128 + 16 * (sbg & 7) + 8 * hh);
    // phase B, slot k: rows 8w + st*RPS2 + rr2 of the block, sub-block g2
    const int g2 = lane % LPR2, rr2 = lane / LPR2, ibB = g2 & 7;
    uint32_t offB[STB];
#pragma unroll
    for (int st = 0; st < STB; ++st)
        offB[st] = (uint32_t)(((ROWS * j + 8 * w + st * RPS2 + rr2) * SBR2 + (g2 >> 3)) * 128 + 16 * ibB);
    // phase B, shared: lane -> row rB of the wave's 8, chunk tB of the XCD's CPX, dword dB
    const int rB = (lane / LPRB) & 7, tB = (lane >> 2) % CPX, dB = lane & 3, ccB = CPX * k + tB;
    const uint32_t offSB = (uint32_t)(((ROWS * j + 8 * w + rB) * SBR2 + (ccB >> 3)) * 128 + 16 * (ccB & 7) + 4 * dB);
    const int hSB = padk(I + 32 * tB) + 4 * dB;
    // The super-block headers a wave needs of one layer, one per lane, fetched by one load
    // (from a few cache lines of the header arrays) and handed to the lanes that use them
    // with ds_bpermute: a load per header set -- every header is shared by 8-16 lanes --
    // would cost address-unit time that the phases' own loads and stores queue behind.
    // Lane order: phase A slot rows (W1, W3 x STA x RPS1 rows x super-blocks), phase A
    // shared rows (2 SRP), phase B slot rows (STB x RPS2 rows x super-blocks), phase B
    // shared rows (8).
    constexpr int NHA = 2 * STA * RPS1 * SBR1, NHS = 2 * SRP, NHB = STB * RPS2 * SBR2;
    static_assert(NHA + NHS + NHB + 8 <= 64, "one header per lane");
    static_assert(SBW <= 8 && 8 % SBW == 0, "a wave's shared K range lies in one super-block");
    int hsel;       // 0 W1, 1 W3, 2/3 shared W1/W3, 4 W2, 5 shared W2
    uint32_t hoff;  // header offset in that matrix
    {
        const int L = lane < NHA + NHS + NHB + 8 ? lane : 0;
        if (L < NHA) {
            const int r = L / SBR1, rr = r % RPS1, st = (r / RPS1) % STA;
            hsel = r / (RPS1 * STA);
            hoff = HDR1 + (uint32_t)(((rowA + st * RPS1 + rr) * SBR1 + L % SBR1) * 8);
        } else if (L < NHA + NHS) {
            const int r = L - NHA;
            hsel = 2 + (r & 1);
            hoff = HDR1 + (uint32_t)(((k * (I / NX) + j * SRP + (r >> 1)) * SBR1 + ((w * SBW) >> 3)) * 8);
        } else if (L < NHA + NHS + NHB) {
            const int r = L - NHA - NHS;
            hsel = 4;
            hoff = HDR2 + (uint32_t)(((ROWS * j + 8 * w + r / SBR2) * SBR2 + r % SBR2) * 8);
        } else {
            hsel = 5;
            hoff = HDR2 + (uint32_t)(((ROWS * j + 8 * w + (L - NHA - NHS - NHB)) * SBR2 + ((CPX * k) >> 3)) * 8);
        }
    }
    // the lanes holding this lane's headers (x4: ds_bpermute byte addresses)
    int hA1[STA], hA3[STA];
#pragma unroll
    for (int st = 0; st < STA; ++st) {
        hA1[st] = 4 * (((0 * STA + st) * RPS1 + rr1) * SBR1 + sb1);
        hA3[st] = 4 * (((1 * STA + st) * RPS1 + rr1) * SBR1 + sb1);
    }
    const int hSA = 4 * (NHA + ri);
    int hB[STB];
#pragma unroll
    for (int st = 0; st < STB; ++st) hB[st] = 4 * (NHA + NHS + (st * RPS2 + rr2) * SBR2 + (g2 >> 3));
    const int hSBr = 4 * (NHA + NHS + NHB + rB);

    // Weights in flight, one set per phase, and the headers of a layer.
    u32x4 aq1[STA], aq3[STA], bq[STB];
    u32x2 saq;
    uint32_t sbq, hd0, hd1;
    // Phase-A weights of the next layer decoded -- codebook bytes and sub-block scales -- while
    // the compute waves would otherwise wait for x (the lookup does not depend on x).
    uint32_t ak1[STA][8], ak3[STA][8], sak[4];
    float as1[STA], as3[STA], sas;
    // ... and this layer's phase-B weights, while the pollers exchange h
    uint32_t bk[STB][8], sbk[2];
    float bs[STB], sbs;

    // Loads of layer li's phase-A (W1, W3) weights for this wave, issued right after phase A
    // of layer li-1 (after B2, so that the routing computed during phase A is visible), and
    // of its phase-B (W2) weights, issued at B1 of layer li: they stream during phase A and
    // the h exchange, which are compute- and L2-bound, and arrive before phase B.  The loads
    // are issued unconditionally -- past the last layer they re-read layer n-1, which is
    // still in the L2 (FETCH_SIZE of a one-layer launch: 18.3 MB = the layer's 15.1 MB, its
    // 2.8 MB of exchange reads and 0.4 MB, not the 10 MB a re-read from HBM would add) --
    // because a conditional burst would make the compiler's load counter
    // path-dependent and turn the waits for the older burst into waits for everything.
    auto prefetch_a = [&](int li) __attribute__((always_inline)) {
        const uint8_t *W1 = rt_p[li % 3][0][0];
        const uint8_t *W3 = rt_p[li % 3][0][1];
        // every header of the layer (phase B's too: used before the next such load) -- AR:
        // requested first, so that each step of phase A waits only for its own rows
        const uint64_t b2 = (uint64_t)rt_p[li % 3][1][0], b3 = (uint64_t)rt_p[li % 3][1][1];
        const uint64_t b4 = (uint64_t)rt_p[li % 3][0][2], b5 = (uint64_t)rt_p[li % 3][1][2];
        uint64_t hb = (uint64_t)W1;
        hb = hsel == 1 ? (uint64_t)W3 : hb;
        hb = hsel == 2 ? b2 : hb;
        hb = hsel == 3 ? b3 : hb;
        hb = hsel == 4 ? b4 : hb;
        hb = hsel == 5 ? b5 : hb;
        u32x2 hd;
        if constexpr (AR) hd = ldg<u32x2>((const uint8_t *)hb + hoff);
#pragma unroll
        for (int st = 0; st < STA; ++st) {
            aq1[st] = ldg<u32x4>(W1 + offA[st]);
            aq3[st] = ldg<u32x4>(W3 + offA[st]);
        }
        saq = ldg<u32x2>(rt_p[li % 3][1][mA] + offSA);
        if constexpr (!AR) hd = ldg<u32x2>((const uint8_t *)hb + hoff);
        hd0 = hd.x;
        hd1 = hd.y;
    };
    auto prefetch_b = [&](int li) __attribute__((always_inline)) {
        const uint8_t *W2 = rt_p[li % 3][0][2];
#pragma unroll
        for (int st = 0; st < STB; ++st) bq[st] = ldg<u32x4>(W2 + offB[st]);
        sbq = ldg<uint32_t>(rt_p[li % 3][1][2] + offSB);
    };
    // the header held by another lane (byte address 4 x lane)
    auto header = [&](int from) __attribute__((always_inline)) {
        return u32x2{(uint32_t)__builtin_amdgcn_ds_bpermute(from, (int)hd0),
                     (uint32_t)__builtin_amdgcn_ds_bpermute(from, (int)hd1)};
    };

    auto decode_a = [&]() __attribute__((always_inline)) {
        // The loaded words pass through empty volatile asm statements, which keep their order
        // with the barrier's: otherwise the compiler may hoist this register-only work above
        // the preceding barrier, onto the critical path.
#pragma unroll
        for (int st = 0; st < STA; ++st) asm volatile("" : "+v"(aq1[st]), "+v"(aq3[st]));
        asm volatile("" : "+v"(saq), "+v"(hd0), "+v"(hd1));
#pragma unroll
        for (int st = 0; st < STA; ++st) {
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                kv_signed8(aq1[st][d], ak1[st][2 * d], ak1[st][2 * d + 1]);
                kv_signed8(aq3[st][d], ak3[st][2 * d], ak3[st][2 * d + 1]);
            }
            as1[st] = sub_scale(header(hA1[st]), ib1);
            as3[st] = sub_scale(header(hA3[st]), ib1);
        }
        kv_signed8(saq[0], sak[0], sak[1]);
        kv_signed8(saq[1], sak[2], sak[3]);
        sas = sub_scale(header(hSA), sbg & 7);
        // ... and the results as well, so that the work is not sunk below the next barrier
        // either
#pragma unroll
        for (int st = 0; st < STA; ++st)
#pragma unroll
            for (int e = 0; e < 8; ++e) asm volatile("" : "+v"(ak1[st][e]), "+v"(ak3[st][e]));
        asm volatile("" : "+v"(sak[0]), "+v"(sak[1]), "+v"(sak[2]), "+v"(sak[3]));
        asm volatile("" : "+v"(as1), "+v"(as3), "+v"(sas));
    };

    // AR: decode_a in pieces, each waiting only for its own loads (the headers, requested
    // first, with the first): step st of the slot rows, then the shared rows
    auto decode_a_step = [&](int st) __attribute__((always_inline)) {
        asm volatile("" : "+v"(aq1[st]), "+v"(aq3[st]), "+v"(hd0), "+v"(hd1));
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            kv_signed8(aq1[st][d], ak1[st][2 * d], ak1[st][2 * d + 1]);
            kv_signed8(aq3[st][d], ak3[st][2 * d], ak3[st][2 * d + 1]);
        }
        as1[st] = sub_scale(header(hA1[st]), ib1);
        as3[st] = sub_scale(header(hA3[st]), ib1);
    };
    auto decode_a_shared = [&]() __attribute__((always_inline)) {
        asm volatile("" : "+v"(saq));
        kv_signed8(saq[0], sak[0], sak[1]);
        kv_signed8(saq[1], sak[2], sak[3]);
        sas = sub_scale(header(hSA), sbg & 7);
    };

    auto decode_b = [&]() __attribute__((always_inline)) {
        // after this wave's phase-A stores ("memory"), for the reason given in decode_a
#pragma unroll
        for (int st = 0; st < STB; ++st) asm volatile("" : "+v"(bq[st]) : : "memory");
        asm volatile("" : "+v"(sbq), "+v"(hd0), "+v"(hd1) : : "memory");
#pragma unroll
        for (int st = 0; st < STB; ++st) {
#pragma unroll
            for (int d = 0; d < 4; ++d) kv_biased8(bq[st][d], bk[st][2 * d], bk[st][2 * d + 1]);
            bs[st] = sub_scale(header(hB[st]), ibB);
        }
        kv_biased8(sbq, sbk[0], sbk[1]);
        sbs = sub_scale(header(hSBr), ccB & 7);
#pragma unroll
        for (int st = 0; st < STB; ++st)
#pragma unroll
            for (int e = 0; e < 8; ++e) asm volatile("" : "+v"(bk[st][e]));
        asm volatile("" : "+v"(sbk[0]), "+v"(sbk[1]), "+v"(bs), "+v"(sbs));
    };

    // AR: this wave's router row of the next layer to route -- row rG, the lane's sub-block
    // g1 (rows past E read row E-1; their logit is a dummy) -- and its element type.  IQ4_XS
    // and f16 weights are requested into registers while the previous layer's x is exchanged;
    // an f32 lane's 128 bytes (one cache line) are only touched then, by one dword load, and
    // read whole by router_dot (from the L2): 32 more registers live across the exchange would
    // spill.
    const int rG = (j * NCW + w) * RPS1 + rr1, rGc = min(rG, a.E - 1);
    u32x4 rq[8];        // IQ4_XS: rq[0] = the 16 qs bytes; f16: rq[0..3]; f32: rq[0..7]
    u32x2 rgh;          // IQ4_XS header
    uint32_t rg_type = MOE_WG_IQ4_XS;
    const uint8_t *rg_row = nullptr; // f32: this lane's 128 bytes
    auto rg_prefetch = [&](int li) __attribute__((always_inline)) {
        const uint64_t *t = reinterpret_cast<const uint64_t *>(a.routers + a.layer0 + li);
        const uint8_t *wg = (const uint8_t *)ldg<uint64_t>(t);
        rg_type = (uint32_t)ldg<uint64_t>(t + 1);
        if (rg_type == MOE_WG_IQ4_XS) {
            const uint8_t *blk = wg + ((size_t)rGc * SBR1 + (g1 >> 3)) * SB_BYTES;
            rgh = ldg<u32x2>(blk);
            const u32x2 q01 = ldg<u32x2>(blk + 8 + 16 * (g1 & 7)), q23 = ldg<u32x2>(blk + 16 + 16 * (g1 & 7));
            rq[0] = u32x4{q01.x, q01.y, q23.x, q23.y};
        } else if (rg_type == MOE_WG_F16) {
            const uint8_t *p = wg + ((size_t)rGc * H + 32 * g1) * 2;
#pragma unroll
            for (int i = 0; i < 4; ++i) rq[i] = ldg<u32x4>(p + 16 * i);
        } else {
            rg_row = wg + ((size_t)rGc * H + 32 * g1) * 4;
            rq[0].x = ldg<uint32_t>(rg_row); // the line into the L2; the value is not used
            asm volatile("" : "+v"(rq[0].x));
        }
    };
    // AR, IQ4_XS: the row's codebook bytes and scale, looked up while x is exchanged (after the
    // row's loads, before B1): router_dot then runs only the dot products
    uint32_t rkv[8];
    float rsc = 0.f;
    auto rg_decode = [&]() __attribute__((always_inline)) {
        if (rg_type == MOE_WG_IQ4_XS) {
            asm volatile("" : "+v"(rq[0]), "+v"(rgh));
#pragma unroll
            for (int d = 0; d < 4; ++d) kv_signed8(rq[0][d], rkv[2 * d], rkv[2 * d + 1]);
            rsc = sub_scale(rgh, g1 & 7);
#pragma unroll
            for (int e = 0; e < 8; ++e) asm volatile("" : "+v"(rkv[e]));
            asm volatile("" : "+v"(rsc));
        }
    };
    // AR: the logit of row rG against x_li (xin = RMSNorm(x) when asked, as phase A), published
    // in this XCD's logit block of layer li
    auto router_dot = [&](int li) __attribute__((always_inline)) {
        uint32_t xh[8], xl[8];
        {
            const u32x4 *c = reinterpret_cast<const u32x4 *>(xq + XQS * g1);
            const u32x4 h0 = c[0], h1 = c[1], l0 = c[2], l1 = c[3];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                xh[e] = h0[e];
                xh[4 + e] = h1[e];
                xl[e] = l0[e];
                xl[4 + e] = l1[e];
            }
        }
        const float sx = xsc[g1];
        const int ab = *abort_lds;
        float inv = 1.0f;
        if (a.rmsnorm) {
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < NSS; ++i) ss += ssq[i];
            inv = __builtin_amdgcn_rsqf(ss * (1.0f / (float)H) + 1e-6f);
        }
        float part;
        if (rg_type == MOE_WG_F32)
#pragma unroll
            for (int i = 0; i < 8; ++i) rq[i] = ldg<u32x4>(rg_row + 16 * i);
        if (rg_type == MOE_WG_IQ4_XS) {
            part = (rsc * sx) * subblock_idot(rkv, xh, xl);
        } else {
            // element 4i + b of the chunk: weight word i, byte / half b; planes dword i, byte
            // b, read biased (xh + 128, by v_cvt_f32_ubyte) with the bias removed once:
            // sum w (xh + xl/256) = sum w (xh + 128) + sum w (xl + 128) / 256 - 128.5 sum w
            float ah = 0.f, al = 0.f, sw = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t bh = xh[i] ^ 0x80808080u, bl = xl[i] ^ 0x80808080u;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const int e = 4 * i + b;
                    float wv;
                    if (rg_type == MOE_WG_F16) {
                        const f16x2 h2 = __builtin_bit_cast(f16x2, (uint32_t)rq[e >> 3][(e >> 1) & 3]);
                        wv = (float)h2[e & 1];
                    } else {
                        wv = __builtin_bit_cast(float, (uint32_t)rq[e >> 2][e & 3]);
                    }
                    ah = __builtin_fmaf(wv, ubyte(bh, b), ah);
                    al = __builtin_fmaf(wv, ubyte(bl, b), al);
                    sw += wv;
                }
            }
            part = sx * (__builtin_fmaf(al, 1.0f / 256.0f, ah) - 128.5f * sw);
        }
        const float tot = inv * row_total<LPR1>(part);
        if (g1 == LPR1_LAST && rG < E4 && !ab) tag_store_local(lbuf(li) + rG, rG < a.E ? tot : 0.0f);
    };

    if constexpr (AR) {
        rg_prefetch(0);
        rg_decode();
    } else {
        prefetch_a(0);
        decode_a();
    }

    for (int li = 0; li < n; ++li) {
        lds_barrier(); // B1: x_l in LDS
        if constexpr (AR) {
            // route this layer from x_l: this wave's logit, then (after BR) the routed
            // experts' weights, requested only now
            router_dot(li);
            lds_barrier(); // BR: routing of li in LDS
            if (w == 0) STK_MARK(STK_EV_ROUTED, li);
            prefetch_a(li);
            __builtin_amdgcn_s_setprio(1);
            __builtin_amdgcn_sched_barrier(0);
            // phase A below decodes and computes step by step as the rows arrive; this layer's
            // W2 rows are requested once the first step's W1/W3 rows are in, not with them (the
            // 9.4 MB of phase A would share the HBM queue with them; phase B needs them only
            // after the h exchange)
        } else {
            // phase A ahead of the other compute wave's decode on this SIMD
            __builtin_amdgcn_s_setprio(1);
            prefetch_b(li);
            __builtin_amdgcn_sched_barrier(0);
        }
        // phase A: h = silu(W1 xin) * (W3 xin) for this wave's slot-k row pairs, and this
        // wave's K share of the workgroup's shared rows (partial g, u: combined by the
        // pollers of every workgroup of the XCD)
        {
            // this lane's chunk (sub-block g1) of x as int8 planes, and its scale
            uint32_t xh[8], xl[8];
            {
                const u32x4 *c = reinterpret_cast<const u32x4 *>(xq + XQS * g1);
                const u32x4 h0 = c[0], h1 = c[1], l0 = c[2], l1 = c[3];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    xh[e] = h0[e];
                    xh[4 + e] = h1[e];
                    xl[e] = l0[e];
                    xl[4 + e] = l1[e];
                }
            }
            const float sx = xsc[g1];
            // a poller whose wait gave up left x invalid (read with the planes: no extra wait)
            const int ab = *abort_lds;
            // shared half sub-block: qs dwords 2hh, 2hh+1 of sub-block sbg
            const uint32_t *cs = xq + XQS * sbg + 2 * hh;
            const u32x2 sxh0 = *reinterpret_cast<const u32x2 *>(cs), sxh1 = *reinterpret_cast<const u32x2 *>(cs + 4);
            const u32x2 sxl0 = *reinterpret_cast<const u32x2 *>(cs + 8), sxl1 = *reinterpret_cast<const u32x2 *>(cs + 12);
            const float ssx = xsc[sbg];
            // RMSNorm scales every activation by one factor, applied to each row's result
            float inv = 1.0f;
            if (a.rmsnorm) {
                float ss = 0.f;
#pragma unroll
                for (int i = 0; i < NSS; ++i) ss += ssq[i];
                inv = __builtin_amdgcn_rsqf(ss * (1.0f / (float)H) + 1e-6f); // v_rsq_f32, 1 ulp
            }
            uint32_t *hb = hbuf(li);
#pragma unroll
            for (int st = 0; st < STA; ++st) {
                if constexpr (AR) {
                    decode_a_step(st);
                    if (st == 0) prefetch_b(li);
                }
                float g = (as1[st] * sx) * subblock_idot(ak1[st], xh, xl);
                float u = (as3[st] * sx) * subblock_idot(ak3[st], xh, xl);
                g = inv * row_total<LPR1>(g);
                u = inv * row_total<LPR1>(u);
                if (g1 == LPR1_LAST && !ab) tag_store_local(hb + rowA + st * RPS1 + rr1, silu_rcp(g) * u);
            }
            if constexpr (AR) decode_a_shared();
            int sah_i = 0, sal_i = 0;
            dword_idot(sak[0], sak[1], sxh0[0], sxh1[0], sxl0[0], sxl1[0], sah_i, sal_i);
            dword_idot(sak[2], sak[3], sxh0[1], sxh1[1], sxl0[1], sxl1[1], sah_i, sal_i);
            float sp = (sas * ssx) * __builtin_fmaf((float)sal_i, 1.0f / 256.0f, (float)sah_i);
            sp = inv * adjacent_sum<LPRS>(sp);
            if (lane % LPRS == 0 && lane < NSA && !ab)
                tag_store_local(hb + I + ((j * SRP + pA) * NCW + w) * 2 + mA, sp);
        }
        __builtin_amdgcn_s_setprio(0);
        if (w == 0) STK_MARK(STK_EV_A, li);
        decode_b();
        lds_barrier(); // B2: h_l in LDS; routing of layer li+2 in LDS
        if (w == 0) STK_MARK(STK_EV_H, li);
        if constexpr (!AR) prefetch_a(min(li + 1, n - 1));
        // nothing of phase B above the burst: its first use of this layer's W2 registers
        // then waits for those loads only, not for everything (stores included) in flight
        __builtin_amdgcn_sched_barrier(0);
        // phase B: W2 rows against h, scaled by c * routing weight
        {
            float hv[32];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                f32x4 q = *reinterpret_cast<const f32x4 *>(hs + padk(32 * g2) + 4 * i);
                hv[4 * i + 0] = q[0];
                hv[4 * i + 1] = q[1];
                hv[4 * i + 2] = q[2];
                hv[4 * i + 3] = q[3];
            }
            const float hsum = hsm[g2];
            const float wk = a.c * rt_w[li % 3][0], wsh = a.c * rt_w[li % 3][1];
#pragma unroll
            for (int st = 0; st < STB; ++st) {
                float d = bs[st] * subblock_dot(bk[st], hv, hsum);
                d = group_sum<LPR2>(d);
                if (g2 == 0) part[0][8 * w + st * RPS2 + rr2] = wk * d;
            }
            float hl[4], hh4[4];
            {
                const f32x4 ql = *reinterpret_cast<const f32x4 *>(hs + hSB);
                const f32x4 qh = *reinterpret_cast<const f32x4 *>(hs + hSB + 16);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    hl[e] = ql[e];
                    hh4[e] = qh[e];
                }
            }
            float ds = sbs * dword_dot(sbk[0], sbk[1], hl, hh4);
            ds = adjacent_sum<LPRB>(ds);
            if (lane % LPRB == 0 && lane < NSB) part[1][8 * w + rB] = wsh * ds;
        }
        if (w == 0) STK_MARK(STK_EV_B, li);
        if constexpr (!AR) {
            // this wave's 8 rows of the XCD's partial (slot k's contribution and its share of
            // the shared expert's) published now, not after B3 by a poller: both parts of a row
            // come from this wave (its own LDS writes, read back in order).  Valid unless a
            // wait of this workgroup gave up (its flag is set before B2 by the waiting wave).
            // Seeded logits: 256.3 -> 255.0 us per token; routed from the activations the
            // poller's publish stays (481 against 498 us with this one).
            asm volatile("" ::: "memory");
            if (lane < 8) {
                const int r = 8 * w + lane;
                const float pv = part[0][r] + part[1][r];
                if (!*abort_lds) tag_store(pbuf(li) + (size_t)k * H + ROWS * j + r, pv);
            }
        }
        lds_barrier(); // B3: every wave past phase B
        // the pollers now gather the partials and exchange x: decode layer li+1's phase-A
        // weights (requested at B2) meanwhile -- or, AR, request layer li+1's router rows
        if constexpr (AR) {
            rg_prefetch(min(li + 1, n - 1));
            rg_decode();
        }
        else decode_a();
    }
}

size_t stack_layer_words(int H, int I) {
    return (size_t)STK_NX * (3 * (size_t)I + (size_t)H + (size_t)(H / 2 + H / 32 + H / 64) + STK_LG_WORDS);
}

template <int H, int I>
static hipError_t launch_stack_t(const StackArgs &a, hipStream_t st, KernelTimer *T) {
    TimedLaunch tl(T, MOE_K_DECODE_STACK, st);
    if (a.logits)
        hipLaunchKernelGGL((k_decode_stack<H, I, false>), dim3(H / 8), dim3(64 * STK_WAVES), 0, st, a);
    else
        hipLaunchKernelGGL((k_decode_stack<H, I, true>), dim3(H / 8), dim3(64 * STK_WAVES), 0, st, a);
    return hipGetLastError();
}

int stack_blocks(int H) { return H / 8; }

template <int H, int I>
static hipError_t stack_occupancy_t(bool ar, int *blocks_per_cu) {
    if (ar)
        return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, k_decode_stack<H, I, true>,
                                                            64 * STK_WAVES, 0);
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, k_decode_stack<H, I, false>, 64 * STK_WAVES,
                                                        0);
}

hipError_t stack_occupancy(int H, int I, bool ar, int *blocks_per_cu) {
    if (H == 2048 && I == 512) return stack_occupancy_t<2048, 512>(ar, blocks_per_cu);
    if (H == 512 && I == 256) return stack_occupancy_t<512, 256>(ar, blocks_per_cu);
    return hipErrorInvalidValue;
}

hipError_t launch_stack(int H, int I, const StackArgs &a, hipStream_t st, KernelTimer *T) {
    if (H == 2048 && I == 512) return launch_stack_t<2048, 512>(a, st, T);
    if (H == 512 && I == 256) return launch_stack_t<512, 256>(a, st, T);
    return hipErrorInvalidValue;
}

} // namespace moe
