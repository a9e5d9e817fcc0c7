// bucket_fill.hpp -- the prefix-sum expert bucket fill as a device body: k_bucket_fill
// (moe_bucket_fill) and the prefill chain's bucket-fill + prep launch (k_pf_route_prep) run it
// in their first 1024-thread workgroup.
#pragma once
#include "moe_internal.hpp"

namespace moe {

// ---------------------------------------------------------------- bucket fill
// Stable counting sort of the 9M (token, slot) pairs into E+1 buckets, replacing the CPU
// loop of src/router.rs:55-97 plus its per-layer upload (src/inference.rs:684-699).
// Tokens are taken 64 at a time (one per lane); inside such a chunk each bucket is a
// 64-bit LDS bitmap of the lanes that named it, so the stable rank of token t inside its
// chunk is popcount(bitmap & lanes-below-t).  Chunk counts get an exclusive scan per
// bucket, the bucket totals a scan over buckets (ranges), and the scatter writes each slot
// to ranges[e] + chunk offset + in-chunk rank: tokens ascend within a bucket, as in the
// reference's cursor fill.  One 1024-thread workgroup; no inter-workgroup synchronisation.
// The same pass writes the grouped-GEMM tile lists (see tile_max_for / stile_max_for).
constexpr int BF_THREADS = 1024;
constexpr int BF_BITMAP_BYTES = 48 * 1024;

__host__ __device__ inline int bucket_cw(int E1) {
    int cw = BF_BITMAP_BYTES / (E1 * 8);
    return cw > 16 ? 16 : (cw < 1 ? 1 : cw);
}
// KEEP: every chunk has its own bitmap set (M <= 64 * bucket_cw): phase 1's bitmaps serve
// phase 3 as they are, and the chunk counts stay in LDS.
__host__ inline size_t bucket_smem(int E1, bool keep) {
    return (size_t)bucket_cw(E1) * E1 * (keep ? 12 : 8) + 5 * (size_t)(E1 + 1) * 4;
}

// Inclusive scan over the wave by DPP: shifts of 1-3 lanes of the original values, then 4 and
// 8 lanes of the partial sums (bank masks keep the lanes whose source is in the same row), then
// row_bcast:15/31 carry the row totals into the rows above -- no LDS round trip.
template <int CTRL, int ROW_MASK, int BANK_MASK>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, BANK_MASK, true);
}
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x) {
    uint32_t s = x + dpp_u<0x111, 0xF, 0xF>(x); // row_shr:1
    s += dpp_u<0x112, 0xF, 0xF>(x);             // row_shr:2
    s += dpp_u<0x113, 0xF, 0xF>(x);             // row_shr:3
    s += dpp_u<0x114, 0xF, 0xE>(s);             // row_shr:4, banks 1-3
    s += dpp_u<0x118, 0xF, 0xC>(s);             // row_shr:8, banks 2-3
    s += dpp_u<0x142, 0xA, 0xF>(s);             // row_bcast:15 into rows 1, 3
    s += dpp_u<0x143, 0xC, 0xF>(s);             // row_bcast:31 into rows 2, 3
    return s;
}

template <bool KEEP>
__device__ __forceinline__ void bucket_fill_body(const BucketArgs &a) {
    extern __shared__ uint32_t smem[];
    __shared__ uint32_t s_flags;
    const int E1 = a.E1, M = a.M;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int nch = (M + 63) / 64;
    const int CW = bucket_cw(E1);
    uint32_t *bm_all = smem;
    // chunk counts [nch][E1]: in LDS after the bitmaps when KEEP, else in global memory
    uint32_t *cnt = KEEP ? smem + (size_t)CW * E1 * 2 : a.chunk_cnt;
    uint32_t *tot = smem + (size_t)CW * E1 * (KEEP ? 3 : 2);
    uint32_t *rg = tot + (E1 + 1);  // bucket starts
    uint32_t *ts = rg + (E1 + 1);   // first full big tile of each bucket
    uint32_t *tp = ts + (E1 + 1);   // partial big tile index (after all full ones)
    uint32_t *tsm = tp + (E1 + 1);  // first small tile
    if (tid == 0) s_flags = 0;
    __syncthreads();
    // Each wave owns one chunk (64 tokens) and one bitmap set at a time, and LDS operations
    // of one wave complete in order, so phases 1 and 3 need no barrier inside.  The first
    // pass keeps its tokens' ids in registers for phase 3.
    uint32_t idk[SLOTS];
    float wk[SLOTS];
    uint32_t okk = 0; // KEEP: bit s = slot s is its token's first naming of the expert
    uint32_t *bm = bm_all + (size_t)(wv < CW ? wv : 0) * E1 * 2;
    const uint32_t bit = 1u << (lane & 31);

    // Phase 1: per-chunk bucket counts.
    for (int base = 0; base < nch; base += CW) {
        const int c = base + wv;
        if (wv < CW && c < nch) {
            for (int i = lane; i < 2 * E1; i += 64) bm[i] = 0;
            const int t = c * 64 + lane;
            uint32_t f = 0;
            if (t < M) {
                uint32_t e9[SLOTS];
#pragma unroll
                for (int s = 0; s < SLOTS; ++s) e9[s] = a.ids[(size_t)t * SLOTS + s];
                if (base == 0)
#pragma unroll
                    for (int s = 0; s < SLOTS; ++s) wk[s] = a.w[(size_t)t * SLOTS + s];
#pragma unroll
                for (int s = 0; s < SLOTS; ++s) {
                    if (base == 0) idk[s] = e9[s];
                    const uint32_t e = e9[s];
                    if (e >= (uint32_t)E1) { f |= MOE_DEVFLAG_BAD_ID; continue; }
                    const uint32_t old = atomicOr(&bm[2 * e + (lane >> 5)], bit);
                    if (old & bit) f |= MOE_DEVFLAG_DUP_ID;
                    else okk |= 1u << s;
                }
            }
            if (f) atomicOr(&s_flags, f);
            for (int e = lane; e < E1; e += 64)
                cnt[(size_t)c * E1 + e] = __popc(bm[2 * e]) + __popc(bm[2 * e + 1]);
        }
    }
    __syncthreads();

    // Phase 2a: exclusive scan of each bucket's chunk counts (in place), bucket totals; the
    // counts are loaded 16 at a time as independent loads before any is overwritten.
    for (int e = tid; e < E1; e += BF_THREADS) {
        uint32_t run = 0;
        for (int c0 = 0; c0 < nch; c0 += 16) {
            uint32_t v[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) v[j] = c0 + j < nch ? cnt[(size_t)(c0 + j) * E1 + e] : 0u;
#pragma unroll
            for (int j = 0; j < 16; ++j)
                if (c0 + j < nch) {
                    cnt[(size_t)(c0 + j) * E1 + e] = run;
                    run += v[j];
                }
        }
        tot[e] = run;
    }
    __syncthreads();

    // Phase 2b: scans over buckets (one wave each): ranges; full big tiles; partial big
    // tiles; small tiles.  Big tiles are listed full ones first, so the long work items
    // start first.
    if (wv < 4) {
        uint32_t *dst = wv == 0 ? rg : (wv == 1 ? ts : (wv == 2 ? tp : tsm));
        uint32_t carry = 0;
        for (int base = 0; base < E1; base += 64) {
            const int e = base + lane;
            const uint32_t n = (e < E1) ? tot[e] : 0u;
            const uint32_t rem = n % PF_BM;
            uint32_t v = n;
            if (wv == 1) v = n / PF_BM;
            else if (wv == 2) v = rem > PF_SMALL_MAX ? 1u : 0u;
            else if (wv == 3) v = (rem > 0 && rem <= PF_SMALL_MAX) ? 1u : 0u;
            const uint32_t inc = wave_incl_scan(v);
            if (e < E1) dst[e] = carry + inc - v;
            carry += (uint32_t)__builtin_amdgcn_readlane((int)inc, 63);
        }
        if (lane == 0) dst[E1] = carry;
    }
    __syncthreads();

    for (int e = tid; e <= E1; e += BF_THREADS) a.ranges[e] = rg[e];
    if (a.tiles) {
        const uint32_t nfull = ts[E1];
        Tile *small = a.tiles + a.tile_max;
        for (int e = tid; e < E1; e += BF_THREADS) {
            const int n = (int)tot[e];
            const int nf = n / PF_BM, rem = n % PF_BM;
            for (int j = 0; j < nf; ++j) a.tiles[ts[e] + j] = Tile{e, (int)rg[e] + j * PF_BM, PF_BM, 0};
            if (rem > PF_SMALL_MAX) {
                a.tiles[nfull + tp[e]] = Tile{e, (int)rg[e] + nf * PF_BM, rem, 0};
            } else if (rem > 0) {
                small[tsm[e]] = Tile{e, (int)rg[e] + nf * PF_BM, rem, 0};
            }
        }
        for (int i = (int)(nfull + tp[E1]) + tid; i < a.tile_max; i += BF_THREADS) a.tiles[i] = Tile{-1, 0, 0, 0};
        for (int i = (int)tsm[E1] + tid; i < a.stile_max; i += BF_THREADS) small[i] = Tile{-1, 0, 0, 0};
    }

    // Phase 3: each chunk's bitmaps (kept from phase 1, or rebuilt) and the scatter.
    for (int base = 0; base < nch; base += CW) {
        const int c = base + wv;
        if (wv < CW && c < nch) {
            if (!KEEP)
                for (int i = lane; i < 2 * E1; i += 64) bm[i] = 0;
            const int t = c * 64 + lane;
            uint32_t ok = KEEP ? okk : 0u;
            uint32_t e9[SLOTS];
            if (t < M) {
#pragma unroll
                for (int s = 0; s < SLOTS; ++s) e9[s] = base == 0 ? idk[s] : (uint32_t)a.ids[(size_t)t * SLOTS + s];
                if (!KEEP)
#pragma unroll
                    for (int s = 0; s < SLOTS; ++s) {
                        if (e9[s] >= (uint32_t)E1) continue;
                        const uint32_t old = atomicOr(&bm[2 * e9[s] + (lane >> 5)], bit);
                        if (!(old & bit)) ok |= 1u << s;
                    }
                const uint32_t below = bit - 1u;
#pragma unroll
                for (int s = 0; s < SLOTS; ++s) {
                    uint32_t p = 0xFFFFFFFFu;
                    if ((ok >> s) & 1u) {
                        const uint32_t e = e9[s];
                        const uint32_t rank = __popc(bm[2 * e + (lane >> 5)] & below) +
                                              ((lane >> 5) ? __popc(bm[2 * e]) : 0u);
                        p = rg[e] + cnt[(size_t)c * E1 + e] + rank;
                        a.sorted_tok[p] = (uint16_t)t;
                        a.sorted_w[p] = base == 0 ? wk[s] : a.w[(size_t)t * SLOTS + s];
                    }
                    if (a.pos) a.pos[(size_t)t * SLOTS + s] = p;
                }
            }
        }
    }
    __syncthreads();
    if (tid == 0 && s_flags) set_flag(a.flags, s_flags);
}

} // namespace moe
