// k_decode.hip -- decode path (M <= 8): IQ4_XS GEMVs over the split weight copy.
//
// Replaces the reference's decode dispatches (src/inference.rs:733-762): per expert a
// w1_w3_fused_m1 GEMV and a w2_scatter_m1 GEMV (shaders/w1_w3_fused_m1.comp,
// shaders/w2_scatter_m1.comp), 18 dispatches and 18 barriers per layer, with SiLU fused
// into the down projection and the combine done as an f16 read-modify-write of the hidden
// state.  Here one layer is two launches, with no waits between workgroups:
//   gate/up item = (pair p, a block of 16 W1/W3 row pairs), where a pair is one (token, slot)
//            of the routing.  The item runs only when p is the first valid pair naming its
//            expert, and then serves every token that named that expert: each selected
//            expert's rows are fetched and decoded once per call, whatever the number of
//            tokens sharing it.  The served tokens' activations are staged in LDS as int8
//            planes (quant4; RMSNorm is one factor per token, applied to the row sums);
//            h = silu(g) * u goes to a [9M][I] f32 scratch.
//   down item = 8 output rows for every token: the waves take the selected experts in turn
//            (each W2 row fetched once per call); every pair's contribution c * w * (W2 h)
//            goes to LDS and a token's 9 contributions are summed in slot order
//            (deterministic, no atomics), the residual added in the same store.
// A single launch with a device-side h exchange between the two roles was built and measured
// (28 us per M = 1 layer against 23 for two launches): every down item needs every expert's
// h, so ~256 workgroups poll and read the same few cache lines past their L2, and memory
// serialises same-address accesses (~11 ns each); a device-scope release fence, the other
// way to publish h, is an L2 writeback here.
// Called with logits (moe_ffn_route, M <= 2), every gate/up workgroup first routes the tokens
// itself -- the top-8 code of moe_router_topk, so all agree bit for bit -- and item 0 publishes
// ids and w for the caller and the down launch (the reference's RouterTopk dispatch + readback
// in do_route, src/inference.rs:608-639, folded into the first launch).
// Pair validity: an id above n_experts, or an id the token already named in an earlier slot,
// drops that slot (MOE_DEVFLAG_BAD_ID / MOE_DEVFLAG_DUP_ID) -- the same slots the prefill
// bucket fill drops, so M = 8 and M = 9 treat such routing alike.
// Lane mapping: a lane owns one 32-weight sub-block of a row: a 16-byte aligned qs load and
// the row's 8-byte header (a row's headers are contiguous in the split layout, so one load
// instruction of a wave touches one cache line of them).
#include "moe_internal.hpp"

namespace moe {

constexpr int DEC_MAXP = MOE_DECODE_MAX_M * SLOTS; // (token, slot) pairs of one call
constexpr int DEC_EMAX = 257;                      // owner table: n_experts <= 256, + shared

struct DecodePlan {
    uint32_t owner[DEC_EMAX]; // first valid pair naming each expert (all ones: none)
    uint64_t valid[2];        // bit q & 63 of word q >> 6: pair q is valid
    uint16_t id[DEC_MAXP];
    float wt[DEC_MAXP];
};

__device__ __forceinline__ bool pair_valid(const DecodePlan &P, int q) { return (P.valid[q >> 6] >> (q & 63)) & 1u; }

// All threads of the workgroup.  The M*9 ids and weights into LDS -- routed here from the
// logits when the call passed them (`publish`: also written out to a.ids / a.w) -- then pair
// validity and each expert's first valid pair.  Returns, in wave 0, the device flags the
// routing raises (0 elsewhere).  Ends with a barrier.
__device__ __forceinline__ uint32_t build_plan(const DecodeArgs &a, DecodePlan &P, bool publish) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, nw = blockDim.x >> 6;
    const int np = a.M * SLOTS;
    if (a.logits && a.M == 1) {
        // One token routed here: its 8 ids are distinct and below E and the shared id is E,
        // so every slot is valid and the only pair naming its expert -- no validity pass,
        // and one LDS-only barrier (the published ids/w are for the next launch).
        if (wv == 0) {
            for (int e = lane; e < DEC_EMAX; e += 64) P.owner[e] = 0xFFFFFFFFu;
            int id;
            float wt;
            route_wave<4>(a.logits, a.E, a.renorm, lane, id, wt);
            if (lane < SLOTS) {
                P.id[lane] = (uint16_t)id;
                P.wt[lane] = wt;
                P.owner[id] = (uint32_t)lane; // after the clear: one wave's LDS writes stay in order
                if (publish) {
                    a.ids[lane] = (uint16_t)id;
                    a.w[lane] = wt;
                }
            }
            if (lane == 0) {
                P.valid[0] = (1ull << SLOTS) - 1;
                P.valid[1] = 0;
            }
        }
        lds_barrier();
        return 0u;
    }
    for (int e = tid; e < DEC_EMAX; e += blockDim.x) P.owner[e] = 0xFFFFFFFFu;
    if (a.logits) {
        for (int t = wv; t < a.M; t += nw) {
            int id;
            float wt;
            route_wave<4>(a.logits + (size_t)t * a.E, a.E, a.renorm, lane, id, wt);
            if (lane < SLOTS) {
                P.id[t * SLOTS + lane] = (uint16_t)id;
                P.wt[t * SLOTS + lane] = wt;
                if (publish) {
                    a.ids[t * SLOTS + lane] = (uint16_t)id;
                    a.w[t * SLOTS + lane] = wt;
                }
            }
        }
    } else {
        for (int q = tid; q < np; q += blockDim.x) {
            P.id[q] = a.ids[q];
            P.wt[q] = a.w[q];
        }
    }
    __syncthreads();
    uint32_t fl = 0;
    if (wv == 0) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int q = lane + 64 * r;
            bool ok = false;
            if (q < np) {
                const int t = q / SLOTS, s = q - t * SLOTS;
                const int e = P.id[q];
                if (e > a.E) {
                    fl |= MOE_DEVFLAG_BAD_ID;
                } else {
                    ok = true;
                    for (int s2 = 0; s2 < s; ++s2) ok = ok && (int)P.id[t * SLOTS + s2] != e;
                    if (ok) atomicMin(&P.owner[e], (uint32_t)q);
                    else fl |= MOE_DEVFLAG_DUP_ID;
                }
            }
            const uint64_t b = __ballot(ok);
            if (lane == 0) P.valid[r] = b;
        }
        fl = (__ballot(fl & MOE_DEVFLAG_BAD_ID) ? MOE_DEVFLAG_BAD_ID : 0u) |
             (__ballot(fl & MOE_DEVFLAG_DUP_ID) ? MOE_DEVFLAG_DUP_ID : 0u);
    }
    __syncthreads();
    return fl;
}

// Wave 0: the pairs q < np for which pred(q) holds, ascending, into list[]; returns their
// number (in wave 0).
template <typename Pred>
__device__ __forceinline__ int collect_pairs(int np, int lane, int *list, Pred pred) {
    int n = 0;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int q = lane + 64 * r;
        const bool m = q < np && pred(q);
        const uint64_t b = __ballot(m);
        if (m) list[n + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u))] = q;
        n += __popcll(b);
    }
    return n;
}


// ---------------------------------------------------------------- roles
// gate/up: 4 waves per workgroup, RP row-pair steps per wave (4 up to M = 2, then 8: fewer
// workgroups, each repeating the routing plan, for the same rows)
constexpr int DEC_ROWS = 8;  // down: output rows per workgroup
template <int H, int I, int RP = 4>
struct DecShape {
    static constexpr int SBR1 = H / QK, LPR1 = SBR1 * 8, RPS1 = 64 / LPR1, RPW1 = RP * RPS1;
    static constexpr int NCHK = I / (4 * RPW1); // gate/up items per pair
    static constexpr int NCH = H / 32;
    static constexpr int SBR2 = I / QK, LPR2 = SBR2 * 8, RPS2 = 64 / LPR2;
    static constexpr int STEPS = DEC_ROWS / RPS2 > 0 ? DEC_ROWS / RPS2 : 1;
    static_assert(LPR1 <= 64 && 64 % LPR1 == 0 && LPR2 <= 64 && 64 % LPR2 == 0, "row must tile a wave");
    static_assert(I % (4 * RPW1) == 0 && RPS2 * STEPS == DEC_ROWS && H % DEC_ROWS == 0, "item shapes");
    static_assert(NCH <= 64, "chunk sums of squares: one per lane");
};

template <int H, int MT>
struct GateUpLds {
    uint32_t xq[MT][(H / 32) * XQS]; // int8 planes per served token
    float xsc[MT][H / 32];           // chunk scales
    float xss[MT][H / 32];           // chunk sums of squares
    int pair[MT];
    int n;
};
struct DownLds {
    float part[DEC_MAXP][DEC_ROWS];
    int first[DEC_MAXP];
    int nf;
};

// ---------------------------------------------------------------- gate/up item
template <int H, int I, int MT, int RP>
__device__ __forceinline__ void gate_up_item(const DecodeArgs &a, const DecodePlan &P, GateUpLds<H, MT> &L, int item) {
    using S = DecShape<H, I, RP>;
    constexpr int SBR = S::SBR1, LPR = S::LPR1, RPS = S::RPS1, RPW = S::RPW1, NCH = S::NCH;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int p = item / S::NCHK, chunk = item - p * S::NCHK;
    const int e = P.id[p];
    if (!pair_valid(P, p) || P.owner[e] != (uint32_t)p) return; // the whole workgroup
    // the pairs this item serves: every valid pair naming e (at most one per token)
    const int np = a.M * SLOTS;
    if (wv == 0) {
        const int n = collect_pairs(np, lane, L.pair, [&](int q) { return pair_valid(P, q) && P.id[q] == e; });
        if (lane == 0) L.n = n;
    }
    lds_barrier();
    const int n = L.n;
    // Loads: this thread's activation chunks (staged below), then the wave's weight rows;
    // the staging waits for the former only.  The barriers up to the compute loop are
    // LDS-only: __syncthreads would also wait for every weight load in flight.
    constexpr int SPT = (MT * NCH + 255) / 256; // chunks per thread
    f32x4 v[SPT][8];
    int kc[SPT];
#pragma unroll
    for (int j = 0; j < SPT; ++j) {
        const int i = tid + 256 * j;
        kc[j] = i < n * NCH ? i : -1;
        if (kc[j] >= 0) {
            const int k = i / NCH, c = i - k * NCH;
            const f32x4 *src = reinterpret_cast<const f32x4 *>(a.x + (size_t)(L.pair[k] / SLOTS) * H + 32 * c);
#pragma unroll
            for (int u = 0; u < 8; ++u) v[j][u] = ldg<f32x4>(src + u);
        }
    }
    const int gsb = lane % LPR, rr = lane / LPR, sb = gsb >> 3, ib = gsb & 7;
    const int rbase = (chunk * 4 + wv) * RPW;
    const uint8_t *W1 = expert_w(a.L.w1, a.L.s1, a.L.sw1, e, a.E);
    const uint8_t *W3 = expert_w(a.L.w3, a.L.s3, a.L.sw3, e, a.E);
    u32x4 q1[RP], q3[RP];
    u32x2 h1[RP], h3[RP];
#pragma unroll
    for (int r = 0; r < RP; ++r) {
        const int row = rbase + r * RPS + rr;
        q1[r] = ldg<u32x4>(W1 + split_qs<SBR>(row, sb) + 16 * ib);
        q3[r] = ldg<u32x4>(W3 + split_qs<SBR>(row, sb) + 16 * ib);
        h1[r] = ldg<u32x2>(W1 + split_hdr<I, SBR>(row, sb));
        h3[r] = ldg<u32x2>(W3 + split_hdr<I, SBR>(row, sb));
    }
    // the activations as int8 planes: one 32-element chunk per thread and step
#pragma unroll
    for (int j = 0; j < SPT; ++j) {
        if (kc[j] < 0) continue;
        const int k = kc[j] / NCH, c = kc[j] - k * NCH;
        float am = 0.f, ss = 0.f;
        bool finite = true;
#pragma unroll
        for (int u = 0; u < 8; ++u)
#pragma unroll
            for (int e4 = 0; e4 < 4; ++e4) {
                const float f = fabsf(v[j][u][e4]);
                finite = finite && f <= 3.4028234e38f;
                am = fmaxf(am, f);
                ss = __builtin_fmaf(v[j][u][e4], v[j][u][e4], ss);
            }
        const float rq = quant_ratio(am);
        uint32_t hw[8], lw[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) quant4(v[j][u], rq, hw[u], lw[u]);
        u32x4 *dst = reinterpret_cast<u32x4 *>(&L.xq[k][c * XQS]);
        dst[0] = u32x4{hw[0], hw[1], hw[2], hw[3]};
        dst[1] = u32x4{hw[4], hw[5], hw[6], hw[7]};
        dst[2] = u32x4{lw[0], lw[1], lw[2], lw[3]};
        dst[3] = u32x4{lw[4], lw[5], lw[6], lw[7]};
        // a non-finite activation makes its chunk's scale NaN, so the rows it meets are NaN
        L.xsc[k][c] = finite ? am * (1.0f / 127.0f) : __builtin_nanf("");
        L.xss[k][c] = ss;
    }
    // codebook bytes and sub-block scales, once for all served tokens
    uint32_t k1[RP][8], k3[RP][8];
    float d1[RP], d3[RP];
#pragma unroll
    for (int r = 0; r < RP; ++r) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            kv_signed8(q1[r][d], k1[r][2 * d], k1[r][2 * d + 1]);
            kv_signed8(q3[r][d], k3[r][2 * d], k3[r][2 * d + 1]);
        }
        d1[r] = sub_scale(h1[r], ib);
        d3[r] = sub_scale(h3[r], ib);
    }
    lds_barrier();
    for (int k = 0; k < n; ++k) {
        float inv = 1.0f;
        if (a.rmsnorm) {
            const float ss = wave_sum(lane < NCH ? L.xss[k][lane] : 0.f);
            inv = 1.0f / sqrtf(ss * (1.0f / (float)H) + 1e-6f);
        }
        const u32x4 *cq = reinterpret_cast<const u32x4 *>(&L.xq[k][gsb * XQS]);
        const u32x4 c0 = cq[0], c1 = cq[1], c2 = cq[2], c3 = cq[3];
        const uint32_t xh[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
        const uint32_t xl[8] = {c2[0], c2[1], c2[2], c2[3], c3[0], c3[1], c3[2], c3[3]};
        const float sx = L.xsc[k][gsb];
        float *hp = a.hbuf + (size_t)L.pair[k] * I + rbase + rr;
#pragma unroll
        for (int r = 0; r < RP; ++r) {
            float g = (d1[r] * sx) * subblock_idot(k1[r], xh, xl);
            float u = (d3[r] * sx) * subblock_idot(k3[r], xh, xl);
            g = inv * row_total<LPR>(g);
            u = inv * row_total<LPR>(u);
            if (gsb == row_total_lane<LPR>()) hp[r * RPS] = silu(g) * u;
        }
    }
}

// ---------------------------------------------------------------- down item
// NW waves per workgroup: 9 at M = 1 (one per selected expert, all loads in flight at once),
// 16 beyond (each wave takes every NW-th expert)
template <int H, int I, int NW>
__device__ __forceinline__ void down_item(const DecodeArgs &a, const DecodePlan &P, DownLds &L, int item) {
    using S = DecShape<H, I>;
    constexpr int SBR = S::SBR2, LPR = S::LPR2, RPS = S::RPS2, STEPS = S::STEPS;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int np = a.M * SLOTS;
    const int n0 = item * DEC_ROWS;
    // the residual this thread adds at the end, requested now (one value per thread)
    float yres = 0.f;
    if (a.accumulate && tid < a.M * DEC_ROWS)
        yres = a.y[(size_t)(tid / DEC_ROWS) * H + n0 + tid % DEC_ROWS];
    // the selected experts: each one's first valid pair, ascending
    if (wv == 0) {
        const int nf = collect_pairs(np, lane, L.first,
                                     [&](int q) { return pair_valid(P, q) && P.owner[P.id[q]] == (uint32_t)q; });
        if (lane == 0) L.nf = nf;
    }
    lds_barrier();
    const int nf = L.nf;
    const int gsb = lane % LPR, rr = lane / LPR, sb = gsb >> 3, ib = gsb & 7;
    for (int u = wv; u < nf; u += NW) {
        const int q0 = L.first[u];
        const int e = P.id[q0];
        // every valid pair naming e, as two 64-bit lane masks
        const uint64_t m0 = __ballot(lane < np && pair_valid(P, lane) && P.id[lane] == e);
        const uint64_t m1 = __ballot(lane + 64 < np && pair_valid(P, lane + 64) && P.id[lane + 64] == e);
        const uint8_t *W2 = expert_w(a.L.w2, a.L.s2, a.L.sw2, e, a.E);
        u32x4 qs[STEPS];
        u32x2 hd[STEPS];
#pragma unroll
        for (int st = 0; st < STEPS; ++st) {
            const int row = n0 + st * RPS + rr;
            qs[st] = ldg<u32x4>(W2 + split_qs<SBR>(row, sb) + 16 * ib);
            hd[st] = ldg<u32x2>(W2 + split_hdr<H, SBR>(row, sb));
        }
        // the first pair's h travels with the weights
        float hv[32];
        load32(a.hbuf + (size_t)q0 * I + 32 * gsb, hv);
        uint32_t kv[STEPS][8];
        float dl[STEPS];
#pragma unroll
        for (int st = 0; st < STEPS; ++st) {
#pragma unroll
            for (int d = 0; d < 4; ++d) kv_biased8(qs[st][d], kv[st][2 * d], kv[st][2 * d + 1]);
            dl[st] = sub_scale(hd[st], ib);
        }
        uint64_t rest[2] = {m0, m1};
        int q = q0;
        while (true) {
            rest[q >> 6] &= ~(1ull << (q & 63));
            float hs = 0.f;
#pragma unroll
            for (int i = 0; i < 32; ++i) hs += hv[i];
            const float wq = a.c * P.wt[q];
#pragma unroll
            for (int st = 0; st < STEPS; ++st) {
                float d = dl[st] * subblock_dot(kv[st], hv, hs);
                d = group_sum<LPR>(d);
                if (gsb == 0) L.part[q][st * RPS + rr] = wq * d;
            }
            if (!(rest[0] | rest[1])) break;
            q = rest[0] ? __builtin_ctzll(rest[0]) : 64 + __builtin_ctzll(rest[1]);
            load32(a.hbuf + (size_t)q * I + 32 * gsb, hv);
        }
    }
    __syncthreads();
    static_assert(MOE_DECODE_MAX_M * DEC_ROWS <= 64 * NW, "one output per thread");
    if (tid < a.M * DEC_ROWS) {
        const int t = tid / DEC_ROWS, r = tid - t * DEC_ROWS;
        float sum = 0.f;
#pragma unroll
        for (int s = 0; s < SLOTS; ++s)
            if (pair_valid(P, t * SLOTS + s)) sum += L.part[t * SLOTS + s][r];
        a.y[(size_t)t * H + n0 + r] = yres + sum;
    }
}

// ---------------------------------------------------------------- down, M = 1
// Wave s takes slot s: it reads the 9 ids itself (no plan, no barrier before the weight
// loads), drops its slot by the rule of build_plan (an id above n_experts, or one an earlier
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
    float yres = 0.f;
    if (a.accumulate && tid < DEC_ROWS) yres = a.y[n0 + tid];
    const int idl = lane < SLOTS ? (int)a.ids[lane] : 0;
    const int e = __builtin_amdgcn_readlane(idl, wv);
    bool ok = e <= a.E;
    for (int s2 = 0; s2 < wv; ++s2) ok = ok && __builtin_amdgcn_readlane(idl, s2) != e;
    const int gsb = lane % LPR, rr = lane / LPR, sb = gsb >> 3, ib = gsb & 7;
    if (ok) {
        const float wq = a.c * a.w[wv];
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
            float d = sub_scale(hd[st], ib) * subblock_dot(kv, hv, hs);
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
// MT: the most tokens one expert can serve in this call (M rounded up to 1, 2, 4, 8).
template <int H, int I, int MT, int RP>
__global__ __launch_bounds__(256) void k_dec_gate_up(DecodeArgs a) {
    __shared__ DecodePlan P;
    __shared__ GateUpLds<H, MT> L;
    const uint32_t fl = build_plan(a, P, blockIdx.x == 0); // ends with a barrier
    if (blockIdx.x == 0 && threadIdx.x == 0 && fl) set_flag(a.flags, fl);
    gate_up_item<H, I, MT, RP>(a, P, L, blockIdx.x);
}

template <int H, int I, int NW>
__global__ __launch_bounds__(64 * NW) void k_dec_down(DecodeArgs a) {
    __shared__ DecodePlan P;
    __shared__ DownLds L;
    (void)build_plan(a, P, false);
    down_item<H, I, NW>(a, P, L, blockIdx.x);
}

template <int H, int I, int MT, int RP>
static void launch_gate_up(const DecodeArgs &a, hipStream_t st) {
    hipLaunchKernelGGL((k_dec_gate_up<H, I, MT, RP>), dim3(a.M * SLOTS * DecShape<H, I, RP>::NCHK), dim3(256), 0, st,
                       a);
}

template <int H, int I>
static hipError_t launch_decode_t(const DecodeArgs &a, hipStream_t st, KernelTimer *T) {
    {
        TimedLaunch tl(T, MOE_K_DECODE_GATE_UP, st);
        if (a.M == 1) launch_gate_up<H, I, 1, 4>(a, st);
        else if (a.M == 2) launch_gate_up<H, I, 2, 4>(a, st);
        else if (a.M <= 4) launch_gate_up<H, I, 4, 8>(a, st);
        else launch_gate_up<H, I, 8, 8>(a, st);
    }
    // the down launch reads the routing from ids/w (published by the gate/up launch when it
    // routed the tokens itself)
    DecodeArgs b = a;
    b.logits = nullptr;
    {
        TimedLaunch tl(T, MOE_K_DECODE_DOWN, st);
        if (a.M == 1) hipLaunchKernelGGL((k_dec_down_m1<H, I>), dim3(H / DEC_ROWS), dim3(64 * SLOTS), 0, st, b);
        else hipLaunchKernelGGL((k_dec_down<H, I, 16>), dim3(H / DEC_ROWS), dim3(1024), 0, st, b);
    }
    return hipGetLastError();
}

hipError_t launch_decode(int H, int I, const DecodeArgs &a, hipStream_t st, KernelTimer *T) {
    if (a.M < 1 || a.M > MOE_DECODE_MAX_M || a.E > DEC_EMAX - 1 || !a.hbuf) return hipErrorInvalidValue;
    if (H == 2048 && I == 512) return launch_decode_t<2048, 512>(a, st, T);
    if (H == 512 && I == 256) return launch_decode_t<512, 256>(a, st, T);
    return hipErrorInvalidValue;
}

} // namespace moe
