// k_decode.hip -- decode path (M <= 8): IQ4_XS GEMVs over the split weight copy.
//
// Replaces the reference's decode dispatches (src/inference.rs:733-762): per expert a
// w1_w3_fused_m1 GEMV and a w2_scatter_m1 GEMV (shaders/w1_w3_fused_m1.comp,
// shaders/w2_scatter_m1.comp), 18 dispatches and 18 barriers per layer, with SiLU fused
// into the down projection and the combine done as an f16 read-modify-write of the hidden
// state.  Here one layer is two launches at M <= 4 and three at 5 <= M <= 8, with no waits
// between workgroups:
//   prep (M >= 5) = one workgroup per token, once per call: its routing when the call passed
//            logits (ids and w are published), its pair validity, its activations as int8
//            planes (quant4) and its RMSNorm factor -- the token's row of a plan block in the
//            scratch.
//   gate/up = one workgroup per CU at M = 1, two beyond.  A step is one W1 row and the same
//            W3 row (16 rows at hidden 512) of one selected expert; wave gw of NW takes
//            steps gw, gw + NW, ..., so every SIMD does an equal share and the shared
//            expert's rows spread over all of them.  Each selected expert's rows are fetched
//            and decoded once per call, whatever the number of tokens sharing it.  At M = 1
//            every wave routes the token itself (the top-8 code of moe_router_topk, so all
//            agree bit for bit) and quantizes x into registers: no plan, no barrier, and the
//            shared expert first in slot order.  Beyond, each workgroup routes the tokens
//            and quantizes their activations into LDS itself (M <= 4: a wave per token) or
//            copies their plan rows (M >= 5), numbers the selected experts in slot order with
//            the tokens each serves, and keeps two rounds of loads in flight.  h = silu(g) * u goes to a
//            [9M][I] f32 scratch.
//   down    = at M = 1, 8 output rows per workgroup, wave s taking slot s; beyond, one
//            workgroup per (token, 8 * MT output rows), the token's h rows quantized into
//            int8 planes in LDS and its (slot, 8-row block) units dealt to eight waves, each
//            requesting all its W2 rows at once (and computing each unit as its rows arrive).  Every pair's contribution c * w * (W2 h)
//            goes to LDS and a token's 9 contributions are summed in slot order
//            (deterministic, no atomics), the residual added in the same store.
// A single launch with a device-side h exchange between the two roles was built and measured
// (28 us per M = 1 layer against 23 for two launches): every down item needs every expert's
// h, so ~256 workgroups poll and read the same few cache lines past their L2, and memory
// serialises same-address accesses (~11 ns each); a device-scope release fence, the other
// way to publish h, is an L2 writeback here.  The routing inside the decode launches stands
// in for the reference's RouterTopk dispatch + readback in do_route
// (src/inference.rs:608-639).
// Pair validity: an id above n_experts, or an id the token already named in an earlier slot,
// drops that slot (MOE_DEVFLAG_BAD_ID / MOE_DEVFLAG_DUP_ID) -- the same slots the prefill
// bucket fill drops, so M = 8 and M = 9 treat such routing alike.
// Lane mapping: a lane owns one 32-weight sub-block of a row: a 16-byte aligned qs load and
// the row's 8-byte header (a row's headers are contiguous in the split layout, so one load
// instruction of a wave touches one cache line of them).
#include <cstddef>

#include "moe_internal.hpp"

namespace moe {

constexpr int DEC_EMAX = 257;                      // owner table: n_experts <= 256, + shared

// The pair rule, the prefill bucket fill's too: slot s of a token is dropped when its id
// exceeds n_experts (MOE_DEVFLAG_BAD_ID) or an earlier slot of the token names the same id
// (MOE_DEVFLAG_DUP_ID).  Lane s < 9 holds slot s's id; returns whether the lane's slot is kept,
// and the wave's flags in fl.
__device__ __forceinline__ bool slot_kept(int id, int lane, int E, uint32_t &fl) {
    bool dup = false;
#pragma unroll
    for (int s2 = 0; s2 < SLOTS - 1; ++s2) dup = dup || (s2 < lane && __builtin_amdgcn_readlane(id, s2) == id);
    fl = (__ballot(lane < SLOTS && id > E) ? MOE_DEVFLAG_BAD_ID : 0u) |
         (__ballot(lane < SLOTS && id <= E && dup) ? MOE_DEVFLAG_DUP_ID : 0u);
    return lane < SLOTS && id <= E && !dup;
}
// The same where the ids may come from the routing inside the launch (routed: wave-uniform):
// routed ids are distinct indices below E and the shared id E, so every slot is kept.
__device__ __forceinline__ bool slot_kept(bool routed, int id, int lane, int E, uint32_t &fl) {
    if (routed) {
        fl = 0u;
        return lane < SLOTS;
    }
    return slot_kept(id, lane, E, fl);
}

// Kernel arguments a launch's chain needs, fetched at the kernel's first instructions: one asm
// takes them all as inputs, so the compiler loads them there in one batch of scalar loads (and
// keeps them in SGPRs; the values, and what the compiler knows of the pointers, are unchanged)
// instead of at a first use deep in the kernel -- where it had placed the layer's pointers
// (after the routing or the plan, in gate/up; after the ids, in down), one more scalar round trip
// on the critical chain.
__device__ __forceinline__ void fetch_gate_up_args(const DecodeArgs &a) {
    asm volatile("" ::"s"(a.L.w1), "s"(a.L.w3), "s"(a.L.s1), "s"(a.L.s3), "s"(a.L.sw1), "s"(a.L.sw3), "s"(a.hbuf),
                 "s"(a.ids), "s"(a.w), "s"(a.flags), "s"(a.plan), "s"(a.M), "s"(a.E), "s"(a.renorm), "s"(a.rmsnorm));
}
__device__ __forceinline__ void fetch_down_args(const DecodeArgs &a) {
    asm volatile("" ::"s"(a.L.w2), "s"(a.L.s2), "s"(a.L.sw2), "s"(a.hbuf), "s"(a.y), "s"(a.ids), "s"(a.w), "s"(a.c),
                 "s"(a.E), "s"(a.accumulate));
}
__device__ __forceinline__ void fetch_prep_args(const DecodeArgs &a) {
    asm volatile("" ::"s"(a.x), "s"(a.logits), "s"(a.ids), "s"(a.w), "s"(a.flags), "s"(a.plan), "s"(a.E),
                 "s"(a.renorm), "s"(a.rmsnorm));
}

// ---------------------------------------------------------------- down shape
constexpr int DEC_ROWS = 8; // down: output rows per workgroup
constexpr int DEC_DOWN_RING = 2; // down, 2 <= M <= 8: units of W2 rows in flight per wave
// Down: a W2 row (I weights) on LPR2 lanes, one 32-weight sub-block per lane; RPS2 rows per
// wave step, STEPS steps for the workgroup's DEC_ROWS rows.
template <int H, int I>
struct DecShape {
    static constexpr int SBR2 = I / QK, LPR2 = SBR2 * 8, RPS2 = 64 / LPR2;
    static constexpr int STEPS = DEC_ROWS / RPS2 > 0 ? DEC_ROWS / RPS2 : 1;
    static_assert(LPR2 <= 64 && 64 % LPR2 == 0, "row must tile a wave");
    static_assert(RPS2 * STEPS == DEC_ROWS && H % DEC_ROWS == 0, "item shapes");
};

// ---------------------------------------------------------------- gate/up
// A step is RPS consecutive row pairs (W1 rows and the same W3 rows) of one selected expert:
// one 16-byte qs piece of each matrix per lane.  The U selected experts are numbered u in
// slot order; expert u owns steps u*SPE .. u*SPE + SPE-1.  Wave gw of the NW = 4 * gridDim.x
// waves takes steps gw, gw + NW, gw + 2 NW, ...: with one workgroup per CU every SIMD gets
// floor or ceil of U*SPE / NW steps, and an expert's rows -- the shared expert's, which serve
// every token, included -- are spread over all waves instead of one workgroup's.
template <int H, int I>
struct GuShape {
    static constexpr int SBR = H / QK, LPR = SBR * 8, RPS = 64 / LPR, SPE = I / RPS, NCH = H / 32;
    static_assert(LPR <= 64 && 64 % LPR == 0 && I % RPS == 0, "a row must tile a wave");
    static_assert(NCH <= 64, "chunk sums of squares: one per lane");
};

// One step's loads for this lane: its qs piece and its super-block header of both matrices.
struct GuLoad {
    u32x4 q1, q3;
    u32x2 h1, h3;
};

template <int H, int I>
__device__ __forceinline__ GuLoad gu_load(const uint8_t *W1, const uint8_t *W3, int row, int sb, int ib) {
    constexpr int SBR = GuShape<H, I>::SBR;
    GuLoad l;
    l.q1 = ldg<u32x4>(W1 + split_qs<SBR>(row, sb) + 16 * ib);
    l.q3 = ldg<u32x4>(W3 + split_qs<SBR>(row, sb) + 16 * ib);
    l.h1 = ldg<u32x2>(W1 + split_hdr<I, SBR>(row, sb));
    l.h3 = ldg<u32x2>(W3 + split_hdr<I, SBR>(row, sb));
    return l;
}

// Signed codebook bytes and sub-block scales of one step's two pieces.
struct GuDec {
    uint32_t k1[8], k3[8];
    float d1, d3;
};

__device__ __forceinline__ void gu_decode(const GuLoad &l, int ib, GuDec &d) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        kv_signed8(l.q1[i], d.k1[2 * i], d.k1[2 * i + 1]);
        kv_signed8(l.q3[i], d.k3[2 * i], d.k3[2 * i + 1]);
    }
    d.d1 = sub_scale(l.h1, ib);
    d.d3 = sub_scale(l.h3, ib);
}

// Row totals of g and u over the LPR lanes of a row in one chain: after the first exchange
// the even lanes carry g and the odd lanes u, and every later level adds lanes of equal parity
// (the other pair of the quad, the row rotated by 4 and by 8, then the gfx950 row swaps), so
// each lane ends with its parity's total.
template <int LPR>
__device__ __forceinline__ float gu_totals(float g, float u, int lane) {
    static_assert(LPR == 16 || LPR == 32 || LPR == 64, "rows of 16, 32 or 64 lanes");
    const bool odd = lane & 1;
    float a = odd ? u : g;
    a += dpp_mov<0xB1>(odd ? g : u); // quad_perm [1,0,3,2]
    a += dpp_mov<0x4E>(a);           // quad_perm [2,3,0,1]
    a += dpp_mov<0x124>(a);          // row_ror:4
    a += dpp_mov<0x128>(a);          // row_ror:8
    if constexpr (LPR >= 32) {
        const auto sw = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, a),
                                                         false, false);
        const uint32_t s0 = sw[0], s1 = sw[1];
        a = __builtin_bit_cast(float, s0) + __builtin_bit_cast(float, s1);
    }
    if constexpr (LPR >= 64) {
        const auto sw = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, a),
                                                         false, false);
        const uint32_t s0 = sw[0], s1 = sw[1];
        a = __builtin_bit_cast(float, s0) + __builtin_bit_cast(float, s1);
    }
    return a;
}

// One (row pair, token): the g and u dots of this lane's sub-block against the token's int8
// planes (scale sx), their row totals, and h = silu(g) * u stored by the row's first lane.
template <int LPR>
__device__ __forceinline__ void gu_row(const GuDec &d, const uint32_t (&xh)[8], const uint32_t (&xl)[8], float sx,
                                       float inv, float *hp, int gsb, int lane) {
    const float g = (d.d1 * sx) * subblock_idot(d.k1, xh, xl);
    const float u = (d.d3 * sx) * subblock_idot(d.k3, xh, xl);
    const float t = inv * gu_totals<LPR>(g, u, lane);
    const float tu = dpp_mov<0xB1>(t); // at an even lane: its odd partner's total, u
    if (gsb == 0) *hp = silu_rcp(t) * tu;
}

// 32 activations (eight quads) -> this chunk's int8 planes, scale (NaN when an activation is
// not finite, so every row it meets is NaN) and sum of squares.
__device__ __forceinline__ void quant_chunk(const f32x4 (&v)[8], uint32_t (&xh)[8], uint32_t (&xl)[8], float &sx,
                                            float &ss) {
    float am = 0.f;
    bool finite = true;
    ss = 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
            const float f = fabsf(v[u][e4]);
            finite = finite && f <= 3.4028234e38f;
            am = fmaxf(am, f);
            ss = __builtin_fmaf(v[u][e4], v[u][e4], ss);
        }
    const float rq = quant_ratio(am);
#pragma unroll
    for (int u = 0; u < 8; ++u) quant4(v[u], rq, xh[u], xl[u]);
    sx = finite ? am * (1.0f / 127.0f) : __builtin_nanf("");
}

__device__ __forceinline__ float rms_factor(int rmsnorm, float ss_wave, int H) {
    return rmsnorm ? 1.0f / sqrtf(ss_wave * (1.0f / (float)H) + 1e-6f) : 1.0f;
}

// ---------------------------------------------------------------- gate/up, M = 1
// No plan: every wave routes the token alone (route_values, the one-wave top-8: the same ids
// and weights as moe_router_topk bit for bit, no LDS, no barrier) or reads the 9 ids; each
// wave checks them by the pair rule, quantizes the lane's chunk of x into registers, and runs
// its steps.  Slot order
// puts the shared expert first: u = 0 is slot 8, u = 1.. the valid routed slots ascending.
// Workgroup 0 publishes the routing (ids and w, for the caller and the down launch) or raises
// the flags of invalid ids.
template <int H, int I>
__global__ __launch_bounds__(256) void k_dec_gate_up_m1(DecodeArgs a) {
    using S = GuShape<H, I>;
    constexpr int LPR = S::LPR, RPS = S::RPS, SPE = S::SPE, NCH = S::NCH;
    constexpr int G = 5; // steps per round of loads (one round with 256 CUs)
    fetch_gate_up_args(a);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gw = (int)blockIdx.x * 4 + wv, NW = (int)gridDim.x * 4;
    const int gsb = lane % LPR, rr = lane / LPR, sb = gsb >> 3, ib = gsb & 7;
    // the token's logit of this lane, then this lane's chunk of x (loads complete in order:
    // the routing waits for the logit only)
    float raw[4] = {0.f, 0.f, 0.f, 0.f};
    if (a.logits) load_logits<4>(a.logits, a.E, lane, raw);
    f32x4 xv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) xv[u] = ldg<f32x4>(a.x + 32 * gsb + 4 * u);
    // routing of the token, by every wave alone (no barrier): lane p < 9 holds slot p
    int id;
    float wt = 1.0f;
    if (a.logits) {
        route_values<4>(raw, a.E, a.renorm, lane, id, wt);
    } else {
        id = lane < SLOTS ? (int)a.ids[lane] : 0;
    }
    uint32_t fl;
    const bool ok = slot_kept(a.logits != nullptr, id, lane, a.E, fl);
    const uint32_t vm = (uint32_t)__ballot(ok) & 0x1FFu;
    if (blockIdx.x == 0 && wv == 0) {
        if (a.logits && lane < SLOTS) {
            a.ids[lane] = (uint16_t)id;
            a.w[lane] = wt;
        }
        if (lane == 0 && fl) set_flag(a.flags, fl);
    }
    // slot order, shared first: bit r of vr = rank position r, slot (r + 8) % 9
    const uint32_t vr = ((vm >> 8) & 1u) | ((vm & 0xFFu) << 1);
    const int U = __builtin_popcount(vm), NS = U * SPE;
    const int nk = gw < NS ? (NS - gw + NW - 1) / NW : 0;
    auto slot_of = [&](int u) __attribute__((always_inline)) {
        uint32_t m = vr;
        if (m != 0x1FFu)
            for (int i = 0; i < u; ++i) m &= m - 1u;
        const int r = m == 0x1FFu ? u : __builtin_ctz(m);
        return r == 0 ? SLOTS - 1 : r - 1;
    };
    uint32_t xh[8], xl[8];
    float sx = 0.f, inv = 1.0f;
    GuLoad ld[G];
    auto issue = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int st = min(gw + (k0 + g) * NW, NS - 1); // past the last step: a valid re-read
            const int u = st / SPE, rs = st - u * SPE;
            const int e = __builtin_amdgcn_readlane(id, slot_of(u));
            ld[g] = gu_load<H, I>(expert_w(a.L.w1, a.L.s1, a.L.sw1, e, a.E),
                                  expert_w(a.L.w3, a.L.s3, a.L.sw3, e, a.E), rs * RPS + rr, sb, ib);
        }
    };
    auto compute = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int st = gw + (k0 + g) * NW;
            if (st >= NS) break;
            const int u = st / SPE, rs = st - u * SPE;
            GuDec d;
            gu_decode(ld[g], ib, d);
            gu_row<LPR>(d, xh, xl, sx, inv, a.hbuf + (size_t)slot_of(u) * I + rs * RPS + rr, gsb, lane);
        }
    };
    if (nk > 0) {
        issue(0);
        // the activations as int8 planes while the weights are in flight.  The barrier keeps
        // this ~500-instruction block (invariant over the rounds) behind the weight requests:
        // the compiler had hoisted it between the routing and the first load (~1 us per call).
        __builtin_amdgcn_sched_barrier(0);
        float ss;
        quant_chunk(xv, xh, xl, sx, ss);
        inv = rms_factor(a.rmsnorm, wave_sum(lane < NCH ? ss : 0.f), H);
        compute(0);
        for (int k0 = G; k0 < nk; k0 += G) {
            issue(k0);
            compute(k0);
        }
    }
}

// ---------------------------------------------------------------- prep, 2 <= M <= 8
// One 4-wave workgroup per token t, once per call: it routes the token when the call passed
// logits (route_wg4, the top-8 of moe_router_topk; ids and w are published) or reads its ids,
// checks its slots by the pair rule (raising the device flags of invalid ids), and quantizes
// its activations into the int8 planes, LPC lanes per 32-element chunk, with its RMSNorm
// factor -- written to the token's rows of the plan block with its valid-slot mask.  The
// logits are requested before the activations, so the routing waits for them only.
template <int H>
__global__ __launch_bounds__(256) void k_dec_prep(DecodeArgs a) {
    using PL = DecPlan<H, MOE_DECODE_MAX_M>;
    constexpr int NCH = H / 32, LPC = 256 / NCH < 8 ? 256 / NCH : 8; // lanes per chunk
    constexpr int QPL = 8 / LPC;                                      // quads per lane
    static_assert(NCH * LPC <= 256 && (LPC & (LPC - 1)) == 0 && QPL >= 1 && QPL <= 2, "chunk lanes");
    __shared__ RouteLds R;
    __shared__ float s_ss[4];
    fetch_prep_args(a);
    PL *P = reinterpret_cast<PL *>(a.plan);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t = blockIdx.x;
    const int c = tid / LPC, p = tid % LPC; // chunk, part of it
    const bool act = c < NCH;
    const float raw = a.logits ? ldg<float>(a.logits + (size_t)t * a.E + min(64 * wv + lane, a.E - 1)) : 0.f;
    f32x4 xv[QPL];
#pragma unroll
    for (int u = 0; u < QPL; ++u)
        xv[u] = ldg<f32x4>(a.x + (size_t)t * H + 32 * min(c, NCH - 1) + 4 * (QPL * p + u));
    int id = 0;
    float wt = 0.f;
    if (a.logits) {
        route_wg4v(raw, a.E, a.renorm, lane, wv, R, id, wt);
        if (wv == 0 && lane < SLOTS) {
            a.ids[t * SLOTS + lane] = (uint16_t)id;
            a.w[t * SLOTS + lane] = wt;
        }
    } else if (wv == 0 && lane < SLOTS) {
        id = (int)a.ids[t * SLOTS + lane];
    }
    if (wv == 0) {
        uint32_t fl;
        const bool ok = slot_kept(a.logits != nullptr, id, lane, a.E, fl);
        const uint32_t vm = (uint32_t)__ballot(ok) & 0x1FFu;
        if (lane == 0) {
            P->vt[t] = vm;
            if (fl) set_flag(a.flags, fl);
        }
    }
    // the chunk's max |x| over its LPC lanes (a non-finite value counts as +inf), the planes
    float am = 0.f, ss = 0.f;
#pragma unroll
    for (int u = 0; u < QPL; ++u)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
            const float f = fabsf(xv[u][e4]);
            am = fmaxf(am, f <= 3.4028234e38f ? f : INFINITY);
            ss = __builtin_fmaf(xv[u][e4], xv[u][e4], ss);
        }
#pragma unroll
    for (int m = 1; m < LPC; m <<= 1) am = fmaxf(am, __shfl_xor(am, m, 64));
    const float rq = quant_ratio(am);
    uint32_t xh[QPL], xl[QPL];
#pragma unroll
    for (int u = 0; u < QPL; ++u) quant4(xv[u], rq, xh[u], xl[u]);
    if (act) {
        uint32_t *dst = &P->xq[t][c * XQS + QPL * p];
        if constexpr (QPL == 2) {
            *reinterpret_cast<u32x2 *>(dst) = u32x2{xh[0], xh[1]};
            *reinterpret_cast<u32x2 *>(dst + 8) = u32x2{xl[0], xl[1]};
        } else {
            dst[0] = xh[0];
            dst[8] = xl[0];
        }
        if (p == 0) P->xsc[t][c] = am <= 3.4028234e38f ? am * (1.0f / 127.0f) : __builtin_nanf("");
    }
    if (a.rmsnorm) {
        const float sw = wave_sum(act ? ss : 0.f);
        if (lane == 0) s_ss[wv] = sw;
        lds_barrier();
        if (tid == 0) P->inv[t] = rms_factor(1, ((s_ss[0] + s_ss[1]) + s_ss[2]) + s_ss[3], H);
    } else if (tid == 0) {
        P->inv[t] = 1.0f;
    }
}

// Maximum over each group of 8 consecutive lanes (non-negative values), in every lane.
__device__ __forceinline__ float group_max8(float v) {
    v = fmaxf(v, dpp_mov<0xB1>(v));  // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_mov<0x4E>(v));  // quad_perm [2,3,0,1]
    return fmaxf(v, dpp_mov<0x141>(v)); // row_half_mirror
}

// Pairs before q (q < 128) set in the two-word mask m.
__device__ __forceinline__ int rank2(uint64_t m0, uint64_t m1, int q) {
    return q < 64 ? __popcll(m0 & ((1ull << q) - 1ull)) : __popcll(m0) + __popcll(m1 & ((1ull << (q - 64)) - 1ull));
}

// ---------------------------------------------------------------- gate/up, 2 <= M <= 8
// INL (M <= 4): each workgroup routes the tokens itself (the top-8 of moe_router_topk, one
// wave per token; workgroup 0 publishes ids, w and the valid-slot masks for the down launch)
// and quantizes their activations into LDS -- no prep launch.  Otherwise (5 <= M <= 8, where
// every workgroup quantizing all the tokens would cost more than the prep launch) it copies
// the tokens' rows of the plan block k_dec_prep wrote and the pairs' ids into LDS (one round
// of loads).  Then it numbers the selected experts in slot order with the tokens each serves
// (so no workgroup waits for another), and each wave runs its steps with two rounds of G
// steps' loads in flight (G = 1: measured faster than 2 to 6 at every M -- with fewer rows in
// flight per wave, each arrives sooner).
template <int H, int I, int MT, bool INL>
__global__ __launch_bounds__(256) void k_dec_gate_up_mt(DecodeArgs a) {
    using S = GuShape<H, I>;
    constexpr int LPR = S::LPR, RPS = S::RPS, SPE = S::SPE, NCH = S::NCH;
    constexpr int G = 1;
    __shared__ DecPlan<H, MT> L;
    __shared__ uint32_t owner[DEC_EMAX]; // first valid pair naming each expert (all ones: none)
    __shared__ uint16_t pid[DEC_MAXP];
    __shared__ float s_ss[MT][4];
    fetch_gate_up_args(a);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gw = (int)blockIdx.x * 4 + wv, NW = (int)gridDim.x * 4;
    const int np = a.M * SLOTS;
    static_assert(DEC_MAXP <= 256, "one pair per thread");
    constexpr int NQ = 8 * NCH, QPT = INL ? MT * NQ / 256 : 1; // quads of a token; per thread
    constexpr int KPT = NQ >= 256 ? NQ / 256 : 1;               // consecutive k of one token
    static_assert(!INL || (MT * NQ % 256 == 0 && NQ % 64 == 0 && QPT % KPT == 0), "a wave's quads are one token's");
    if constexpr (INL) {
        constexpr int TPW = (MT + 3) / 4; // tokens routed per wave
        auto *P = reinterpret_cast<DecPlan<H, MOE_DECODE_MAX_M> *>(a.plan);
        // Loads, all unconditional (so the compiler's counts of the in-order loads stay exact):
        // the logits of this wave's tokens wv, wv + 4 (x stands in when there are none) and
        // their ids (read when not routing), then quad tid + 256 k of the M x NQ activation
        // quads (threads past the last re-read it): the routing waits for its own loads alone.
        float raw[TPW][4];
        int idr[TPW];
        static_assert(H >= DEC_EMAX - 1, "x stands in for the logits: M x H >= M x E floats");
        const float *lg = a.logits ? a.logits : a.x;
#pragma unroll
        for (int r = 0; r < TPW; ++r) {
            const int t = min(wv + 4 * r, a.M - 1);
            load_logits<4>(lg + (size_t)t * a.E, a.E, lane, raw[r]);
            idr[r] = (int)a.ids[t * SLOTS + min(lane, SLOTS - 1)];
        }
        f32x4 xv[QPT];
#pragma unroll
        for (int k = 0; k < QPT; ++k) xv[k] = ldg<f32x4>(a.x + 4 * min(tid + 256 * k, a.M * NQ - 1));
        for (int e = tid; e < DEC_EMAX; e += 256) owner[e] = 0xFFFFFFFFu;
        if (tid < DEC_MAXP) L.tmask[tid] = 0u;
        // routing, the pair rule and the valid-slot masks of this wave's tokens; workgroup 0
        // publishes them (the masks for the down launch) and raises the flags of invalid ids
#pragma unroll
        for (int r = 0; r < TPW; ++r) {
            const int t = wv + 4 * r;
            if (t >= a.M) break;
            int id = lane < SLOTS ? idr[r] : 0;
            float wt = 0.f;
            if (a.logits) route_values<4>(raw[r], a.E, a.renorm, lane, id, wt);
            uint32_t fl;
            const bool ok = slot_kept(a.logits != nullptr, id, lane, a.E, fl);
            const uint32_t vm = (uint32_t)__ballot(ok) & 0x1FFu;
            if (lane < SLOTS) pid[t * SLOTS + lane] = (uint16_t)id;
            if (lane == 0) L.vt[t] = vm;
            if (blockIdx.x == 0) {
                if (a.logits && lane < SLOTS) {
                    a.ids[t * SLOTS + lane] = (uint16_t)id;
                    a.w[t * SLOTS + lane] = wt;
                }
                if (lane == 0) {
                    P->vt[t] = vm;
                    if (fl) set_flag(a.flags, fl);
                }
            }
        }
        // The activations as int8 planes: quad q = tid + 256 k is elements 4 (q % 8) .. + 3 of
        // chunk (q / 8) % NCH of token q / NQ (one token per wave and k), the chunk maximum
        // over its 8 lanes; each wave's sum of squares of each token (0 for tokens it holds
        // no quad of).
        if (lane == 0)
#pragma unroll
            for (int t = 0; t < MT; ++t) s_ss[t][wv] = 0.f;
#pragma unroll
        for (int k0 = 0; k0 < QPT; k0 += KPT) {
            float ss = 0.f;
            const int t = __builtin_amdgcn_readfirstlane((tid + 256 * k0) / NQ);
#pragma unroll
            for (int k = k0; k < k0 + KPT; ++k) {
                const int q = tid + 256 * k, c = (q / 8) % NCH, p = q % 8;
                float am = 0.f;
#pragma unroll
                for (int e4 = 0; e4 < 4; ++e4) {
                    const float f = fabsf(xv[k][e4]);
                    am = fmaxf(am, f <= 3.4028234e38f ? f : INFINITY);
                    ss = __builtin_fmaf(xv[k][e4], xv[k][e4], ss);
                }
                am = group_max8(am);
                uint32_t xh, xl;
                quant4(xv[k], quant_ratio(am), xh, xl);
                if (t < a.M) {
                    L.xq[t][c * XQS + p] = xh;
                    L.xq[t][c * XQS + 8 + p] = xl;
                    if (p == 0) L.xsc[t][c] = am <= 3.4028234e38f ? am * (1.0f / 127.0f) : __builtin_nanf("");
                }
            }
            const float sw = wave_sum(ss);
            if (lane == 0 && t < a.M) s_ss[t][wv] = sw;
        }
    } else {
        constexpr int XQR = NCH * XQS * 4, XSR = NCH * 4;
        constexpr int PLB = 8 * MOE_DECODE_MAX_M + MT * (XQR + XSR); // plan bytes this launch copies
        constexpr int CPT = (PLB / 16 + 255) / 256;                     // 16-byte pieces per thread
        // the tokens' factors and valid-slot masks, the M rows of planes and the M rows of
        // scales (global rows are MOE_DECODE_MAX_M apart, local ones MT), and the pairs' ids:
        // all loads in flight, then the stores
        using LP = DecPlan<H, MT>;
        constexpr int H0 = (int)offsetof(LP, inv), HL = (int)offsetof(LP, uexp) - H0;
        static_assert(H0 % 16 == 0 && HL == 8 * MOE_DECODE_MAX_M, "head rows of whole 16-byte pieces");
        const uint8_t *src = reinterpret_cast<const uint8_t *>(a.plan);
        uint8_t *dst = reinterpret_cast<uint8_t *>(&L);
        const int nq = HL / 16 + a.M * (XQR + XSR) / 16;
        u32x4 cv[CPT];
        int co[CPT];
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int k = min(tid + 256 * j, nq - 1);
            int gi, li; // byte offsets
            if (k < HL / 16) {
                gi = li = H0 + 16 * k;
            } else if (k < HL / 16 + a.M * XQR / 16) {
                gi = li = (int)DEC_PLAN_HEAD + 16 * k - HL;
            } else {
                const int r = 16 * k - HL - a.M * XQR;
                gi = (int)DEC_PLAN_HEAD + MOE_DECODE_MAX_M * XQR + r;
                li = (int)DEC_PLAN_HEAD + MT * XQR + r;
            }
            co[j] = tid + 256 * j < nq ? li : -1;
            cv[j] = ldg<u32x4>(src + gi);
        }
        const int idq = tid < np ? (int)a.ids[tid] : 0;
        for (int e = tid; e < DEC_EMAX; e += 256) owner[e] = 0xFFFFFFFFu;
        if (tid < DEC_MAXP) L.tmask[tid] = 0u;
#pragma unroll
        for (int j = 0; j < CPT; ++j)
            if (co[j] >= 0) *reinterpret_cast<u32x4 *>(dst + co[j]) = cv[j];
        if (tid < np) pid[tid] = (uint16_t)idq;
    }
    __syncthreads();
    if (INL && tid < a.M) L.inv[tid] = rms_factor(a.rmsnorm, ((s_ss[tid][0] + s_ss[tid][1]) + s_ss[tid][2]) + s_ss[tid][3], H);
    // each expert's first valid pair, then wave 0 numbers the selected experts in slot order
    // with the tokens each serves and their pairs
    if (tid < np && ((L.vt[tid / SLOTS] >> (tid % SLOTS)) & 1u)) atomicMin(&owner[pid[tid]], (uint32_t)tid);
    __syncthreads();
    if (wv == 0) {
        int idr[2];
        bool vq[2], own[2];
        uint32_t ow[2];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int q = lane + 64 * r;
            vq[r] = q < np && ((L.vt[min(q / SLOTS, MT - 1)] >> (q % SLOTS)) & 1u);
            idr[r] = vq[r] ? (int)pid[q] : 0;
            ow[r] = vq[r] ? owner[idr[r]] : 0u;
            own[r] = vq[r] && ow[r] == (uint32_t)q;
        }
        const uint64_t om0 = __ballot(own[0]), om1 = __ballot(own[1]);
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            if (!vq[r]) continue;
            const int q = lane + 64 * r, tq = q / SLOTS;
            const int u = rank2(om0, om1, (int)ow[r]); // the slot-order number of q's expert
            atomicOr(&L.tmask[u], 1u << tq);
            L.tpair[u][tq] = (uint8_t)q;
            if (own[r]) L.uexp[u] = idr[r];
        }
        if (lane == 0) L.U = __popcll(om0) + __popcll(om1);
    }
    __syncthreads();
    const int gsb = lane % LPR, rr = lane / LPR, sb = gsb >> 3, ib = gsb & 7;
    const int NS = L.U * SPE;
    const int nk = gw < NS ? (NS - gw + NW - 1) / NW : 0;
    const int nit = (nk + G - 1) / G;
    if (nit == 0) return;
    auto issue = [&](GuLoad (&ld)[G], int it) __attribute__((always_inline)) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int st = min(gw + (it * G + g) * NW, NS - 1); // past the last step: a valid re-read
            const int u = st / SPE, rs = st - u * SPE;
            const int e = L.uexp[u];
            ld[g] = gu_load<H, I>(expert_w(a.L.w1, a.L.s1, a.L.sw1, e, a.E),
                                  expert_w(a.L.w3, a.L.s3, a.L.sw3, e, a.E), rs * RPS + rr, sb, ib);
        }
    };
    auto compute = [&](const GuLoad (&ld)[G], int it) __attribute__((always_inline)) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int st = gw + (it * G + g) * NW;
            if (st >= NS) break;
            const int u = st / SPE, rs = st - u * SPE;
            GuDec d;
            gu_decode(ld[g], ib, d);
            uint32_t tm = L.tmask[u];
            while (tm) {
                const int t = __builtin_ctz(tm);
                tm &= tm - 1u;
                const u32x4 *cq = reinterpret_cast<const u32x4 *>(&L.xq[t][gsb * XQS]);
                const u32x4 c0 = cq[0], c1 = cq[1], c2 = cq[2], c3 = cq[3];
                const uint32_t xh[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
                const uint32_t xl[8] = {c2[0], c2[1], c2[2], c2[3], c3[0], c3[1], c3[2], c3[3]};
                gu_row<LPR>(d, xh, xl, L.xsc[t][gsb], L.inv[t], a.hbuf + (size_t)L.tpair[u][t] * I + rs * RPS + rr,
                            gsb, lane);
            }
        }
    };
    GuLoad A[G], B[G];
    issue(A, 0);
    issue(B, 1);
    int it = 0;
    for (; it + 2 < nit; it += 2) {
        compute(A, it);
        issue(A, it + 2);
        compute(B, it + 1);
        issue(B, it + 3);
    }
    compute(A, it);
    compute(B, it + 1);
}

// ---------------------------------------------------------------- down, 2 <= M <= 8
// Token-major: workgroup (t, b) writes output rows b*R .. b*R + R-1 (R = 8 * MT) of token t.
// Its units are (k-th valid slot of t, 8-row block j of the R): the slot's expert's W2 rows
// against the pair's h, times c * w, into LDS; units are dealt to the eight waves in turn and
// a wave requests the W2 rows of all its units at once.  The token's 9 h rows are quantized
// into int8 planes in LDS, one 32-element chunk per lane, exactly as gate/up stages its
// activations (their loads issued before the W2 rows), so a sub-block dot is 16
// v_dot4_i32_i8.  The slot sums then run in slot order with the residual.  Workgroup index
// t * NRB + b: with NRB a multiple of 8 every token's copy of row block b sits on one XCD, so
// the W2 rows of an expert two tokens share (the shared expert's always) are read from HBM
// once and are L2 hits for the other tokens.
template <int H, int I, int MT>
__global__ __launch_bounds__(512) void k_dec_down_mt(DecodeArgs a) {
    using S = DecShape<H, I>;
    using PL = DecPlan<H, MOE_DECODE_MAX_M>;
    constexpr int SBR = S::SBR2, LPR = S::LPR2, RPS = S::RPS2, STEPS = S::STEPS;
    constexpr int NWV = 8, R = DEC_ROWS * MT, NRB = H / R, MAXU = (SLOTS * MT + NWV - 1) / NWV;
    constexpr int CPR = I / 32, NCK = SLOTS * CPR; // h chunks per row, of the token
    static_assert(I % 32 == 0 && CPR == LPR, "one h chunk per W2 sub-block lane");
    static_assert(NCK <= 64 * NWV && R <= 64 * NWV && H % R == 0, "one chunk, one output per thread");
    __shared__ __attribute__((aligned(16))) uint32_t xq[NCK * XQS];
    __shared__ float xs[NCK];
    __shared__ float part[SLOTS][R];
    const PL *P = reinterpret_cast<const PL *>(a.plan);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t = (int)blockIdx.x / NRB, n0 = ((int)blockIdx.x % NRB) * R;
    // The token's valid slots (bit s of vt): lane k < nvs takes the k-th one's slot ks, and its
    // expert and weight are requested first, the h chunks next, the W2 rows last: the W2 loads
    // wait for the ids alone, the quantization for h alone, and each unit below for its own
    // rows.  Every load is unconditional (threads and units past the last one re-read a valid
    // address), so the compiler's counts of the in-order loads stay exact at every wait.
    const uint32_t vt = __builtin_amdgcn_readfirstlane(P->vt[t]);
    const int nvs = __popc(vt), nun = nvs * MT;
    uint32_t vm = vt;
#pragma unroll
    for (int i = 0; i < SLOTS - 1; ++i)
        if (i < lane) vm &= vm - 1u;
    const int ks = lane < nvs ? __builtin_ctz(vm) : 0;
    const int ke = (int)a.ids[t * SLOTS + ks];
    const float kw = a.w[t * SLOTS + ks];
    // chunk tid of the token's 9 h rows (row s chunk c is chunk s * CPR + c)
    f32x4 hv[8];
    {
        const float *src = a.hbuf + (size_t)t * SLOTS * I + 32 * min(tid, NCK - 1);
#pragma unroll
        for (int u = 0; u < 8; ++u) hv[u] = ldg<f32x4>(src + 4 * u);
    }
    const float yv = a.y[(size_t)t * H + n0 + min(tid, R - 1)];
    const float yres = a.accumulate && tid < R ? yv : 0.f;
    const int nu = nun > wv ? (nun - wv + NWV - 1) / NWV : 0; // this wave's units wv, wv + 8, ...
    const int gsb = lane % LPR, rr = lane / LPR, sb = gsb >> 3, ib = gsb & 7;
    // W2 rows of unit i of this wave (past the last unit, or with no valid slot, the shared
    // expert's: a valid re-read), in a ring of DR units: unit i + DR is requested once unit i
    // is done.  Fewer rows in flight per wave finish sooner each (measured: all nine units of
    // M = 8 requested at once arrive together, late).
    constexpr int DR = MAXU < DEC_DOWN_RING ? MAXU : DEC_DOWN_RING;
    u32x4 qs[DR][STEPS];
    u32x2 hd[DR][STEPS];
    auto issue_unit = [&](int i) __attribute__((always_inline)) {
        const int j = max(min(wv + NWV * i, nun - 1), 0);
        const int e = nun > 0 ? __builtin_amdgcn_readlane(ke, j / MT) : a.E;
        const uint8_t *W2 = expert_w(a.L.w2, a.L.s2, a.L.sw2, e, a.E);
#pragma unroll
        for (int st = 0; st < STEPS; ++st) {
            const int row = n0 + (j % MT) * DEC_ROWS + st * RPS + rr;
            qs[i % DR][st] = ldg<u32x4>(W2 + split_qs<SBR>(row, sb) + 16 * ib);
            hd[i % DR][st] = ldg<u32x2>(W2 + split_hdr<H, SBR>(row, sb));
        }
    };
#pragma unroll
    for (int i = 0; i < DR; ++i) issue_unit(i);
    if (tid < NCK) {
        uint32_t h8[8], l8[8];
        float sx, ss;
        quant_chunk(hv, h8, l8, sx, ss);
        u32x4 *dst = reinterpret_cast<u32x4 *>(&xq[tid * XQS]);
        dst[0] = u32x4{h8[0], h8[1], h8[2], h8[3]};
        dst[1] = u32x4{h8[4], h8[5], h8[6], h8[7]};
        dst[2] = u32x4{l8[0], l8[1], l8[2], l8[3]};
        dst[3] = u32x4{l8[4], l8[5], l8[6], l8[7]};
        xs[tid] = sx;
    }
    lds_barrier();
#pragma unroll
    for (int i = 0; i < MAXU; ++i) {
        if (i < nu) {
            const int j = wv + NWV * i, k = j / MT;
            const int s = __builtin_amdgcn_readlane(ks, k);
            const float cw = a.c * __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, kw), k));
            // the pair's chunk gsb as planes
            const int c = s * CPR + gsb;
            const u32x4 *cq = reinterpret_cast<const u32x4 *>(&xq[c * XQS]);
            const u32x4 c0 = cq[0], c1 = cq[1], c2 = cq[2], c3 = cq[3];
            const uint32_t xh[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
            const uint32_t xl[8] = {c2[0], c2[1], c2[2], c2[3], c3[0], c3[1], c3[2], c3[3]};
            const float sx = xs[c];
#pragma unroll
            for (int st = 0; st < STEPS; ++st) {
                uint32_t kv[8];
#pragma unroll
                for (int d = 0; d < 4; ++d) kv_signed8(qs[i % DR][st][d], kv[2 * d], kv[2 * d + 1]);
                float d = sub_scale(hd[i % DR][st], ib) * sx * subblock_idot(kv, xh, xl);
                d = group_sum<LPR>(d);
                if (gsb == 0) part[s][(j % MT) * DEC_ROWS + st * RPS + rr] = cw * d;
            }
        }
        if (i + DR < MAXU) issue_unit(i + DR);
    }
    __syncthreads();
    if (tid < R) {
        float sum = 0.f;
#pragma unroll
        for (int s = 0; s < SLOTS; ++s)
            if ((vt >> s) & 1u) sum += part[s][tid];
        a.y[(size_t)t * H + n0 + tid] = yres + sum;
    }
}

// ---------------------------------------------------------------- down, M = 1
// Wave s takes slot s: it reads the 9 ids itself (no plan, no barrier before the weight
// loads), drops its slot by the pair rule (an id above n_experts, or one an earlier
// slot names), and writes c * w_s * (W2_e h_s) for the workgroup's 8 output rows to LDS; the
// 9 contributions are then summed in slot order with the residual.
template <int H, int I>
__global__ __launch_bounds__(64 * SLOTS) void k_dec_down_m1(DecodeArgs a) {
    using S = DecShape<H, I>;
    constexpr int SBR = S::SBR2, LPR = S::LPR2, RPS = S::RPS2, STEPS = S::STEPS;
    __shared__ float part[SLOTS][DEC_ROWS];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n0 = blockIdx.x * DEC_ROWS;
    fetch_down_args(a);
    float yres = 0.f;
    if (a.accumulate && tid < DEC_ROWS) yres = a.y[n0 + tid];
    const int idl = lane < SLOTS ? (int)a.ids[lane] : 0;
    // the slot's weight requested beside the ids (the weight rows wait for the ids, not for it)
    const float wsl = ldg<float>(a.w + wv);
    const int e = __builtin_amdgcn_readlane(idl, wv);
    bool ok = e <= a.E;
    for (int s2 = 0; s2 < wv; ++s2) ok = ok && __builtin_amdgcn_readlane(idl, s2) != e;
    const int gsb = lane % LPR, rr = lane / LPR, sb = gsb >> 3, ib = gsb & 7;
    if (ok) {
        const float wq = a.c * wsl;
        const uint8_t *W2 = expert_w(a.L.w2, a.L.s2, a.L.sw2, e, a.E);
        u32x4 qs[STEPS];
        u32x2 hd[STEPS];
#pragma unroll
        for (int st = 0; st < STEPS; ++st) {
            const int row = n0 + st * RPS + rr;
            qs[st] = ldg<u32x4>(W2 + split_qs<SBR>(row, sb) + 16 * ib);
            hd[st] = ldg<u32x2>(W2 + split_hdr<H, SBR>(row, sb));
        }
        float hv[32];
        load32(a.hbuf + (size_t)wv * I + 32 * gsb, hv);
        float hs = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) hs += hv[i];
#pragma unroll
        for (int st = 0; st < STEPS; ++st) {
            uint32_t kv[8];
#pragma unroll
            for (int d = 0; d < 4; ++d) kv_biased8(qs[st][d], kv[2 * d], kv[2 * d + 1]);
            float d = sub_scale(hd[st], ib) * subblock_dot_mix(kv, hv, hs);
            d = group_sum<LPR>(d);
            if (gsb == 0) part[wv][st * RPS + rr] = wq * d;
        }
    } else if (lane < DEC_ROWS) {
        part[wv][lane] = 0.f;
    }
    lds_barrier();
    if (tid < DEC_ROWS) {
        float sum = 0.f;
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) sum += part[s][tid];
        a.y[n0 + tid] = yres + sum;
    }
}

// ---------------------------------------------------------------- the launches
using DecPlanBig = DecPlan<2048, 8>;
using DecPlanSmall = DecPlan<512, 2>;
static_assert(offsetof(DecPlanBig, xq) == DEC_PLAN_HEAD && offsetof(DecPlanSmall, xq) == DEC_PLAN_HEAD,
              "plan head layout");
static_assert(sizeof(DecPlan<DEC_MAX_H, MOE_DECODE_MAX_M>) <= decode_plan_floats(DEC_MAX_H) * 4, "plan block size");

template <int H, int I>
static hipError_t launch_decode_t(const DecodeArgs &a, hipStream_t st, KernelTimer *T) {
    // M >= 2: the prep launch routes (when given logits) and publishes ids/w, so the later
    // launches read the routing from ids/w and the plan block
    DecodeArgs b = a;
    if (a.M > 4) {
        TimedLaunch tl(T, MOE_K_DECODE_PREP, st);
        hipLaunchKernelGGL((k_dec_prep<H>), dim3(a.M), dim3(256), 0, st, a);
        b.logits = nullptr;
    }
    {
        TimedLaunch tl(T, MOE_K_DECODE_GATE_UP, st);
        const dim3 grid((unsigned)a.nwg), blk(256);
        if (a.M == 1) hipLaunchKernelGGL((k_dec_gate_up_m1<H, I>), grid, blk, 0, st, a);
        else if (a.M == 2) hipLaunchKernelGGL((k_dec_gate_up_mt<H, I, 2, true>), grid, blk, 0, st, a);
        else if (a.M <= 4) hipLaunchKernelGGL((k_dec_gate_up_mt<H, I, 4, true>), grid, blk, 0, st, a);
        else hipLaunchKernelGGL((k_dec_gate_up_mt<H, I, 8, false>), grid, blk, 0, st, b);
    }
    // the down launch reads the routing from ids/w (published by the first launch when it
    // routed the tokens itself)
    b.logits = nullptr;
    {
        TimedLaunch tl(T, MOE_K_DECODE_DOWN, st);
        if (a.M == 1) hipLaunchKernelGGL((k_dec_down_m1<H, I>), dim3(H / DEC_ROWS), dim3(64 * SLOTS), 0, st, b);
        else if (a.M == 2) hipLaunchKernelGGL((k_dec_down_mt<H, I, 2>), dim3(a.M * H / (DEC_ROWS * 2)), dim3(512), 0, st, b);
        else if (a.M <= 4) hipLaunchKernelGGL((k_dec_down_mt<H, I, 4>), dim3(a.M * H / (DEC_ROWS * 4)), dim3(512), 0, st, b);
        else hipLaunchKernelGGL((k_dec_down_mt<H, I, 8>), dim3(a.M * H / (DEC_ROWS * 8)), dim3(512), 0, st, b);
    }
    return hipGetLastError();
}

hipError_t launch_decode(int H, int I, const DecodeArgs &a, hipStream_t st, KernelTimer *T) {
    if (a.M < 1 || a.M > MOE_DECODE_MAX_M || a.E > DEC_EMAX - 1 || !a.hbuf || a.nwg < 1 || (a.M >= 2 && !a.plan))
        return hipErrorInvalidValue;
    if (H == 2048 && I == 512) return launch_decode_t<2048, 512>(a, st, T);
    if (H == 512 && I == 256) return launch_decode_t<512, 256>(a, st, T);
    return hipErrorInvalidValue;
}

} // namespace moe
