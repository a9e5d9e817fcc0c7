// bucket_fill.hpp -- the prefix-sum expert bucket fill as device bodies, run by
// moe_bucket_fill (k_route.hip) and by the prefill chain's first launches (k_prefill.hip).
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
// reference's cursor fill.  Up to 16 chunks (1024 tokens) one 1024-thread workgroup does it
// all; beyond that the chunks are spread over workgroups (bucket_count_chunk, bucket_scan_wg,
// bucket_scatter_chunk).
// The same pass writes the grouped-GEMM tile lists (see tile_max_for).
constexpr int BF_THREADS = 1024;
constexpr int BF_BITMAP_BYTES = 48 * 1024;

__host__ __device__ inline int bucket_cw(int E1) {
    int cw = BF_BITMAP_BYTES / (E1 * 8);
    return cw > 16 ? 16 : (cw < 1 ? 1 : cw);
}
// keep: the one-workgroup fill (M <= 64 * bucket_cw, chunk counts in LDS); else the
// many-workgroup scan launch.
__host__ __device__ inline size_t bucket_smem(int E1, bool keep) {
    return (size_t)bucket_cw(E1) * E1 * (keep ? 12 : 8) + 5 * (size_t)(E1 + 1) * 4;
}
// The one-workgroup fill also stages the sorted weights and tokens of its 9M slots in LDS.
__host__ inline size_t bucket_smem_one(int E1, int M) { return bucket_smem(E1, true) + (size_t)SLOTS * M * 6; }

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

// ---- per-chunk pieces (one wave, one 64-token chunk)

// Chunk c's bucket bitmaps in bm (two words per bucket: lanes 0-31, 32-63), built from the
// ids of its tokens, which are left in e9.  ok bit s: slot s is its token's first naming of
// an id below E1.  Returns the MOE_DEVFLAG bits seen.  LDS operations of one wave complete
// in order, so no barrier is needed between the clear and the atomics.
__device__ __forceinline__ uint32_t chunk_bitmaps(const BucketArgs &a, uint32_t *bm, int c, int lane,
                                                  uint32_t (&e9)[SLOTS], uint32_t &ok) {
    const int E1 = a.E1, t = c * 64 + lane;
    const uint32_t bit = 1u << (lane & 31);
    for (int i = lane; i < 2 * E1; i += 64) bm[i] = 0;
    uint32_t f = 0;
    ok = 0;
    if (t < a.M) {
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) e9[s] = a.ids[(size_t)t * SLOTS + s];
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) {
            const uint32_t e = e9[s];
            if (e >= (uint32_t)E1) { f |= MOE_DEVFLAG_BAD_ID; continue; }
            const uint32_t old = atomicOr(&bm[2 * e + (lane >> 5)], bit);
            if (old & bit) f |= MOE_DEVFLAG_DUP_ID;
            else ok |= 1u << s;
        }
    }
    return f;
}

// Chunk counts live at cnt[c * CL.cs + e * CL.es] ([chunk][bucket] in LDS or global memory).
struct CntLayout {
    uint32_t *cnt;
    int cs, es;
    __device__ uint32_t &at(int c, int e) const { return cnt[(size_t)c * cs + (size_t)e * es]; }
};

__device__ __forceinline__ void chunk_counts(const uint32_t *bm, CntLayout CL, int c, int E1, int lane) {
    for (int e = lane; e < E1; e += 64) CL.at(c, e) = __popc(bm[2 * e]) + __popc(bm[2 * e + 1]);
}

// Scatter of chunk c: slot (t, s) goes to rg[e] + (chunk offset of c in bucket e) + (rank of
// t among the chunk's tokens naming e).  wk: the slot weights when already in registers, else
// read here.  Every load is issued before the first store (the stores could alias them as
// far as the compiler knows, which would otherwise serialise nine round trips).
// otok, ow: where the sorted tokens and weights go (the caller's arrays, or LDS staging).
template <typename TokPtr, typename WPtr>
__device__ __forceinline__ void chunk_scatter(const BucketArgs &a, const uint32_t *bm, const uint32_t *rg,
                                              CntLayout CL, int c, int lane, const uint32_t (&e9)[SLOTS],
                                              uint32_t ok, const float *wk, TokPtr otok, WPtr ow) {
    const int t = c * 64 + lane;
    if (t >= a.M) return;
    const uint32_t bit = 1u << (lane & 31), below = bit - 1u;
    uint32_t p[SLOTS];
    float wv[SLOTS];
    // loads outside any branch (a load under a divergent branch makes the waits count
    // conservatively, one round trip per slot); dropped slots read bucket 0 and are discarded
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
        const bool on = (ok >> s) & 1u;
        const uint32_t e = on ? e9[s] : 0u;
        const uint32_t rank = __popc(bm[2 * e + (lane >> 5)] & below) + ((lane >> 5) ? __popc(bm[2 * e]) : 0u);
        const uint32_t q = rg[e] + CL.at(c, (int)e) + rank;
        wv[s] = wk ? wk[s] : a.w[(size_t)t * SLOTS + s];
        p[s] = on ? q : 0xFFFFFFFFu;
    }
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
        if (p[s] != 0xFFFFFFFFu) {
            otok[p[s]] = (uint16_t)t;
            ow[p[s]] = wv[s];
        }
        if (a.pos) a.pos[(size_t)t * SLOTS + s] = p[s];
    }
}

// ---- whole-workgroup pieces

// LDS scratch after the bitmaps: bucket totals, starts and the tile-list scans.
struct BucketScan {
    uint32_t *tot, *rg, *ts, *tp, *tsm;
};
__device__ __forceinline__ BucketScan bucket_scan_lds(uint32_t *p, int E1) {
    return BucketScan{p, p + (E1 + 1), p + 2 * (E1 + 1), p + 3 * (E1 + 1), p + 4 * (E1 + 1)};
}

// Phase 2b and the lists, from the bucket totals in S.tot: scans over buckets (ranges, tile
// counts) into S, and -- when write -- the ranges and the tile lists to global memory.  Every
// thread of the workgroup; ends with a barrier.
__device__ __forceinline__ void bucket_lists(const BucketArgs &a, BucketScan S, bool write) {
    const int E1 = a.E1;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    // 2b: scans over buckets (one wave each): ranges; full big tiles; partial big tiles;
    // small tiles.  Big tiles are listed full ones first, so the long work items start first.
    if (wv < 4) {
        uint32_t *dst = wv == 0 ? S.rg : (wv == 1 ? S.ts : (wv == 2 ? S.tp : S.tsm));
        uint32_t carry = 0;
        for (int base = 0; base < E1; base += 64) {
            const int e = base + lane;
            const uint32_t n = (e < E1) ? S.tot[e] : 0u;
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

    if (write)
        for (int e = tid; e <= E1; e += BF_THREADS) a.ranges[e] = S.rg[e];
    if (write && a.tiles) {
        // one list: full tiles, big remainders, then small remainders, then empty entries up to
        // tile_max (every expert has at most one remainder, so the tiles never exceed it)
        const uint32_t nfull = S.ts[E1], nbig = nfull + S.tp[E1];
        Tile *small = a.tiles + nbig;
        for (int e = tid; e < E1; e += BF_THREADS) {
            const int n = (int)S.tot[e];
            const int nf = n / PF_BM, rem = n % PF_BM;
            for (int j = 0; j < nf; ++j) a.tiles[S.ts[e] + j] = Tile{e, (int)S.rg[e] + j * PF_BM, PF_BM, 0};
            if (rem > PF_SMALL_MAX) {
                a.tiles[nfull + S.tp[e]] = Tile{e, (int)S.rg[e] + nf * PF_BM, rem, 0};
            } else if (rem > 0) {
                small[S.tsm[e]] = Tile{e, (int)S.rg[e] + nf * PF_BM, rem, 0};
            }
        }
        for (int i = (int)(nbig + S.tsm[E1]) + tid; i < a.tile_max; i += BF_THREADS) a.tiles[i] = Tile{-1, 0, 0, 0};
    }
    __syncthreads();
}

// Phases 2a/2b and the lists: exclusive scan of each bucket's chunk counts in place, bucket
// totals, ranges, and the tile lists.  Every thread of the workgroup; ends with a barrier.
// 2a loads B counts at a time as independent loads before any is overwritten (B = 16: with 64
// the chunks' uniform offsets took 128 SGPRs, 112 of them spilled).
template <int B>
__device__ __forceinline__ void bucket_scan_and_lists(const BucketArgs &a, CntLayout CL, int nch, BucketScan S) {
    const int E1 = a.E1;
    const int tid = threadIdx.x;
    for (int e = tid; e < E1; e += BF_THREADS) {
        uint32_t run = 0;
        for (int c0 = 0; c0 < nch; c0 += B) {
            uint32_t v[B];
            // every load unconditional (the index clamped, the value dropped below)
#pragma unroll
            for (int j = 0; j < B; ++j) v[j] = CL.at(c0 + j < nch ? c0 + j : nch - 1, e);
#pragma unroll
            for (int j = 0; j < B; ++j)
                if (c0 + j < nch) {
                    CL.at(c0 + j, e) = run;
                    run += v[j];
                }
        }
        S.tot[e] = run;
    }
    __syncthreads();
    bucket_lists(a, S, true);
}

// ---- one workgroup, at most bucket_cw(E1) chunks: every chunk has its own bitmap set (one
// wave each), the counts stay in LDS, and the scatter reuses the bitmaps, ids and weights
// of the counting pass.  The scatter writes the sorted weights and tokens into LDS and the
// workgroup then stores them in order: one CU's 2 x 9M scattered 2- and 4-byte global stores
// took ~3.7 us at M = 512, the LDS scatter and the coalesced copy a fraction of that.
__device__ __forceinline__ void bucket_fill_one_wg(const BucketArgs &a) {
    extern __shared__ uint32_t smem[];
    __shared__ uint32_t s_flags;
    const int E1 = a.E1;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int nch = (a.M + 63) / 64, CW = bucket_cw(E1);
    const CntLayout CL{smem + (size_t)CW * E1 * 2, E1, 1}; // [nch][E1] in LDS
    const BucketScan S = bucket_scan_lds(smem + (size_t)CW * E1 * 3, E1);
    float *st_w = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(smem) + bucket_smem(E1, true));
    uint16_t *st_tok = reinterpret_cast<uint16_t *>(st_w + (size_t)SLOTS * a.M);
    if (tid == 0) s_flags = 0;
    __syncthreads();
    const int c = wv;
    const bool mine = wv < CW && c < nch;
    uint32_t *bm = smem + (size_t)(mine ? wv : 0) * E1 * 2;
    uint32_t e9[SLOTS] = {}, ok = 0;
    float wk[SLOTS] = {};
    if (mine) {
        const uint32_t f = chunk_bitmaps(a, bm, c, lane, e9, ok);
        if (f) atomicOr(&s_flags, f);
        if (c * 64 + lane < a.M)
#pragma unroll
            for (int s = 0; s < SLOTS; ++s) wk[s] = a.w[(size_t)(c * 64 + lane) * SLOTS + s];
        chunk_counts(bm, CL, c, E1, lane);
    }
    __syncthreads();
    bucket_scan_and_lists<16>(a, CL, nch, S); // nch <= 16
    if (mine) chunk_scatter(a, bm, S.rg, CL, c, lane, e9, ok, wk, st_tok, st_w);
    __syncthreads();
    const int nv = (int)S.rg[E1]; // valid slots
    for (int i = tid; i < nv; i += BF_THREADS) {
        a.sorted_tok[i] = st_tok[i];
        a.sorted_w[i] = st_w[i];
    }
    if (tid == 0 && s_flags) set_flag(a.flags, s_flags);
}

__host__ __device__ inline bool bucket_one_wg(int M, int E1) { return (M + 63) / 64 <= bucket_cw(E1); }

// ---- many workgroups (large M): three launches -- count (one 64-thread workgroup per
// chunk), scan (one 1024-thread workgroup: the chunk offsets, ranges and lists), scatter (one
// workgroup per chunk, rebuilding its bitmaps).  One chunk per CU-resident workgroup spreads
// the scattered 2- and 4-byte accesses over many CUs' address units.  The launch boundaries
// order the steps; no workgroup waits for another.  Same result as the one-workgroup fill,
// slot for slot.
constexpr int BF_CHUNK_THREADS = 64;
__host__ inline size_t bucket_chunk_smem(int E1) { return (size_t)(2 * E1 + E1 + 1) * 4; }
__device__ __forceinline__ CntLayout bucket_global_cnt(const BucketArgs &a) {
    return CntLayout{a.chunk_cnt, a.E1, 1}; // [nch][E1]
}

__device__ __forceinline__ void bucket_count_chunk(const BucketArgs &a, int c) {
    extern __shared__ uint32_t smem[];
    const int lane = threadIdx.x;
    uint32_t e9[SLOTS], ok;
    const uint32_t f = chunk_bitmaps(a, smem, c, lane, e9, ok);
    if (f) set_flag(a.flags, f); // only for invalid ids
    chunk_counts(smem, bucket_global_cnt(a), c, a.E1, lane);
}

__device__ __forceinline__ void bucket_scan_wg(const BucketArgs &a) {
    extern __shared__ uint32_t smem[];
    bucket_scan_and_lists<16>(a, bucket_global_cnt(a), (a.M + 63) / 64, bucket_scan_lds(smem, a.E1));
}

__device__ __forceinline__ void bucket_scatter_chunk(const BucketArgs &a, int c) {
    extern __shared__ uint32_t smem[];
    const int E1 = a.E1, lane = threadIdx.x;
    uint32_t *bm = smem, *rg = smem + 2 * E1;
    for (int e = lane; e <= E1; e += 64) rg[e] = a.ranges[e];
    uint32_t e9[SLOTS], ok;
    (void)chunk_bitmaps(a, bm, c, lane, e9, ok); // one wave: LDS operations complete in order
    chunk_scatter(a, bm, rg, bucket_global_cnt(a), c, lane, e9, ok, nullptr, a.sorted_tok, a.sorted_w);
}

} // namespace moe
