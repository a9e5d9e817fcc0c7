// moe_internal.hpp -- launcher declarations and argument blocks shared by the .hip units.
#pragma once

#include "moe_device.hpp"
#include "moe_ffn.h"

namespace moe {

// Grouped-GEMM tile: rows [row0, row0+nrows) of the expert-sorted slot order, all of
// expert `expert`.  expert < 0 marks an unused entry of the fixed-size launch grid.
struct Tile {
    int32_t expert, row0, nrows, pad;
};

constexpr int PF_BM = 64;  // prefill big-tile rows (token slots of one expert)
constexpr int PF_SMALL_MAX = 32; // remainders of at most this many slots are listed as small tiles
// h columns per prefill gate/up work item, and per hmax block: 64 (two waves per 16 columns,
// alternate K stages: half-length items, which fill the last round of workgroup slots better)
// for M <= PF_SPLIT_MAX_M, else 128 (one wave per 16 columns: fewer items to stage A for).
// Measured (H 2048, I 512): split 121.8 / wide 127.4 us at M = 512; 184.6 / 175.8 at 1024.
constexpr int PF_NGU = 64;
constexpr int PF_NGU_WIDE = 128;
constexpr int PF_SPLIT_MAX_M = 768;

struct DecodeArgs {
    LayerPtrs L;          // split copy of the layer (k_repack_split)
    const float *x;
    const float *logits;  // non-null: the gate/up launch routes the tokens and publishes ids, w
    uint16_t *ids;        // [M][9] (read, or written when logits is set)
    float *w;             // [M][9]
    float *y;
    float *hbuf;          // [9M][I] f32 h scratch
    uint32_t *flags;      // sticky device flags
    int M, E, accumulate, rmsnorm, renorm;
    float c;
    int nwg;              // gate/up workgroups (a multiple of the CU count)
    void *plan;           // 2 <= M <= 8: the plan block (DecPlan<H, MOE_DECODE_MAX_M>) after hbuf
};

constexpr int DEC_MAXP = MOE_DECODE_MAX_M * SLOTS; // (token, slot) pairs of one decode call

// Plan block of the 2 <= M <= 8 decode launches.  In the scratch k_dec_prep writes each
// token's row: its RMSNorm factor, its valid slots, and its activations as int8 planes with
// their chunk scales.  Every gate/up workgroup copies those rows into an LDS DecPlan<H, MT>
// and fills the rest of the head itself: the selected experts in slot order (each one's first
// valid pair ascending), the tokens each serves and their pairs.
template <int H, int MT>
struct DecPlan {
    int U;                                     // selected experts (LDS copy only)
    int pad_[3];
    float inv[MOE_DECODE_MAX_M];               // RMSNorm factor per token
    uint32_t vt[MOE_DECODE_MAX_M];             // valid slots per token (bit s)
    int uexp[DEC_MAXP];                        // expert id of selected expert u (LDS copy only)
    uint32_t tmask[DEC_MAXP];                  // tokens it serves (LDS copy only)
    uint8_t tpair[DEC_MAXP][MOE_DECODE_MAX_M]; // ... and each one's pair (LDS copy only)
    uint32_t xq[MT][(H / 32) * XQS]; // int8 planes per token (chunk c at XQS * c)
    float xsc[MT][H / 32];           // chunk scales
};
constexpr size_t DEC_PLAN_HEAD = 16 + 8 * MOE_DECODE_MAX_M + 8 * DEC_MAXP + DEC_MAXP * MOE_DECODE_MAX_M;
static_assert(DEC_PLAN_HEAD % 16 == 0, "plan rows start 16-byte aligned");
constexpr size_t DEC_MAX_H = 2048; // the largest hidden size the decode kernels are built for
// Floats of the decode path's scratch: h [9 * MOE_DECODE_MAX_M][I] f32, then the plan block.
constexpr size_t decode_hbuf_floats(size_t I) { return (size_t)DEC_MAXP * I; }
constexpr size_t decode_plan_floats(size_t H) {
    return (DEC_PLAN_HEAD + MOE_DECODE_MAX_M * (H / 32) * (XQS + 1) * 4 + 255) / 256 * 64;
}
inline size_t decode_scratch_floats(int H, int I) {
    return decode_hbuf_floats((size_t)I) + decode_plan_floats((size_t)H);
}

struct BucketArgs {
    const uint16_t *ids;
    const float *w;
    int M, E1; // E1 = n_experts + 1 buckets
    uint32_t *ranges;     // [E1+1]
    uint16_t *sorted_tok; // [9M]
    float *sorted_w;      // [9M]
    uint32_t *pos;        // [M][9] or null
    uint32_t *chunk_cnt;  // workspace: ceil(M/64) * E1 chunk counts
    Tile *tiles;          // [tile_max]: full tiles, big remainders, small remainders, empty; or null
    int tile_max;
    uint32_t *flags;
};

// The prefill chain's own bucket fill (k_pf_count, k_pf_place): slots placed by an atomic rank
// inside their bucket, not in token order -- no row of the GEMMs depends on its position, so
// the output is the same bit for bit -- in two launches of many workgroups.
struct PfCountArgs {
    const float *logits; // [M][E]: routed here into ids / w; null: ids / w given
    uint16_t *ids;       // [M][9]
    float *w;            // [M][9]
    int M, E, renorm;
    uint32_t *cnt;       // [E + 1] bucket counters: zero on entry (k_pf_combine zeroes them)
    uint32_t *slot;      // [9M] (bucket << 23) | rank in the bucket, or ~0 for a dropped slot
    uint32_t *flags;
};
constexpr int PF_SLOT_RANK_BITS = 23; // a slot's expert above these bits
constexpr int PF_CNT_COPIES = 8;      // striped bucket counters (one per XCD)
constexpr int PF_SLOT_COPY_SHIFT = 20; // its counter copy at bits 20..22, its rank below: ranks < 9 * 65535 < 2^20

// Prefill reads the split copy of a layer (k_repack_split), as the decode kernels do.
struct PrefillArgs {
    LayerPtrs L;
    const float *x;
    _Float16 *xh;        // [M][H] f16: x (normalised if requested) * s_t, K permuted in 32-blocks
    float *xinv;         // [M] 1 / s_t (s_t a power of two)
    const uint16_t *sorted_tok;
    const float *sorted_w;
    const uint32_t *pos; // [M][9]
    const Tile *tiles;
    _Float16 *hh;        // [9M][I] h = silu(g) * u as f16, sorted slot order: each PF_NGU-column
                         // block scaled by the power of two of its max (hmax), K order of the
                         // down kernel's A (perm32_pos inside 32-column blocks)
    float *hmax;         // [9M][I/PF_NGU] max |h| per row and PF_NGU-column block
    _Float16 *part;      // [9M][H] c*w-scaled expert outputs in sorted slot order, as f16
                         // times 2^pexp per 32-column block; columns n and 16 + n of a block
                         // stored side by side
    int8_t *pexp;        // [9M][H/32] those exponents
    float *y;
    int M, E, accumulate, rmsnorm, tile_max;
    float c;
    uint32_t *cnt;       // the fill's bucket counters: zeroed by k_pf_combine for the next call
};

constexpr int STK_CWAVES = 8;             // decode stack: 8 compute waves (two per SIMD),
constexpr int STK_WAVES = STK_CWAVES + 3; // 1 router wave, 2 poller waves

// A layer's router gate matrix as bound by moe_bind_router: [E][H] of element type `type`
// (MOE_WG_*) in the caller's memory; wg null when none is bound.
struct StackRouter {
    const uint8_t *wg;
    uint32_t type, pad;
};
static_assert(sizeof(StackRouter) == 16, "router table entry");

struct StackArgs {
    const LayerPtrs *layers; // device table indexed by absolute layer
    const StackRouter *routers; // device table indexed by absolute layer (activation routing)
    int layer0, n_layers;
    const float *x;          // [H] input activation
    const float *logits;     // [n_layers][E], or null: every layer routed from its input (routers)
    float *y;                // [H] output activation (may alias x)
    uint16_t *ids_out;       // [n_layers][9] or null
    float *w_out;            // [n_layers][9] or null
    // Two sets of tagged exchange buffers, set_words words each (n_max layer blocks of
    // stack_layer_words(H, I)): a launch uses set (epoch & 1), which the previous launch
    // cleared, and clears the other one for the next launch.
    uint32_t *xs;
    size_t set_words;
    int n_max;               // layer blocks per set (the context's n_layers)
    uint32_t *ctl;           // control words, STK_CTL_STRIDE apart (STK_CTL_*)
    uint32_t *flags;         // [0] sticky device flags, [1] abort word (tagged with the epoch)
    uint32_t spin_max;       // poll rounds before a bounded wait expires
    int E, rmsnorm, renorm;
    float c;
    uint64_t *trace;         // -DMOE_STACK_TRACE builds: [NB][n_layers][STK_TRACE_EV] clocks, or null
};
constexpr int STK_TRACE_EV = 16; // words per (workgroup, layer) of a stack trace

constexpr uint32_t STK_SPIN_DEFAULT = 1u << 16;
// Control words of the decode stack, each on its own 128-byte line: one workgroup ticket
// counter per XCD, the count of last-layer reducers done and of those that left (XCD 0), the
// launch epoch (its parity picks the exchange set) and the number of layer blocks each set
// may hold written words in.  All zero at moe_create and after a recovery.
constexpr int STK_CTL_STRIDE = 32;
constexpr int STK_CTL_DONE = 8, STK_CTL_EXIT = 9, STK_CTL_EPOCH = 10, STK_CTL_DIRTY = 11; // DIRTY + set
constexpr int STK_CTL_WORDS = 16 * STK_CTL_STRIDE;

// Optional per-kernel timing (moe_timing_enable): each launch is bracketed by two HIP
// events recorded on the launch's own stream.  Events are created when timing is enabled,
// never inside a hot call.
struct KernelTimer {
    hipEvent_t *ev = nullptr; // 2 * cap events
    int *kid = nullptr;       // kernel id of each pair
    int cap = 0, n = 0, dropped = 0;
};

struct TimedLaunch {
    KernelTimer *T;
    hipStream_t st;
    bool on;
    TimedLaunch(KernelTimer *t, int id, hipStream_t s) : T(t), st(s), on(false) {
        if (T && T->cap > 0) {
            if (T->n < T->cap) {
                T->kid[T->n] = id;
                on = hipEventRecord(T->ev[2 * T->n], st) == hipSuccess;
            } else {
                T->dropped++;
            }
        }
    }
    ~TimedLaunch() {
        if (on && hipEventRecord(T->ev[2 * T->n + 1], st) == hipSuccess) T->n++;
    }
};

hipError_t launch_dequant(const void *blocks, uint64_t n_sb, float *out, hipStream_t st);
// Decode-stack copy of a layer: per matrix, the 128-byte qs of every super-block, then its
// 8-byte headers, same order (k_repack_split).
hipError_t launch_repack_split(const void *src, uint64_t src_stride, const void *shared, void *dst,
                               uint64_t dst_stride, int E, int rows, int cols, hipStream_t st);
hipError_t launch_gen_iq4xs(void *dst, uint64_t n, uint64_t seed, uint64_t first, hipStream_t st);
hipError_t launch_gen_normal(float *dst, uint64_t n, uint64_t seed, uint64_t first, float mean,
                             float stdv, hipStream_t st);
hipError_t launch_gen_logits(float *dst, int M, int E, uint64_t seed, int kind, double param,
                             double hot_value, hipStream_t st);
hipError_t launch_router_topk(const float *logits, int M, int E, int renorm, uint16_t *ids,
                              float *w, hipStream_t st, KernelTimer *T);
hipError_t launch_bucket_fill(const BucketArgs &a, hipStream_t st, KernelTimer *T);
// Router gate GEMV on Wg of type wtype (MOE_WG_*), then -- with ids -- the top-8 (a
// k_router_topk launch).
hipError_t launch_router_gemv(int H, int wtype, const void *wg, const float *x, int M, int E, int rmsnorm,
                              float *logits, int renorm, uint16_t *ids, float *w, hipStream_t st, KernelTimer *T);
hipError_t launch_decode(int H, int I, const DecodeArgs &a, hipStream_t st, KernelTimer *T);
// prep, one gate/up and one down launch over both tile lists, combine -- all on st.
// Bucket fill and prep (one launch), gate/up, down, combine.
hipError_t launch_prefill(int H, int I, const BucketArgs &b, const PfCountArgs &c, const PrefillArgs &a,
                          hipStream_t st, KernelTimer *T);
hipError_t launch_stack(int H, int I, const StackArgs &a, hipStream_t st, KernelTimer *T);
// *dst = the sticky device flags, which are cleared (stream ordered).  When they hold
// MOE_DEVFLAG_TIMEOUT, the decode stack's state -- `stack_words` words from `stack` on, its
// control words and both exchange sets -- is zeroed as well (recovery after an expired wait).
hipError_t launch_flags_take(uint32_t *flags, uint32_t *dst, uint32_t *stack, size_t stack_words, hipStream_t st);
// ar: the activation-routed form of the kernel (StackArgs::logits null).
hipError_t stack_occupancy(int H, int I, bool ar, int *blocks_per_cu);
int stack_blocks(int H);
// Words of one layer block of a decode-stack exchange set: per XCD the h words (3I), the
// partial of every output row (H), x' as int8 pair words + chunk scales + per-workgroup
// sums of squares (H/2 + H/32 + H/64), and the layer's router logits (STK_LG_WORDS, used by
// the activation-routed form only).
constexpr int STK_LG_WORDS = 256;
size_t stack_layer_words(int H, int I);

// Tiles: the PF_BM-slot tiles of every expert, then each expert's remainder (above
// PF_SMALL_MAX slots a big tile, else a small one): at most one remainder per expert.
inline int tile_max_for(int M, int E1) { return (9 * M + PF_BM - 1) / PF_BM + E1; }

} // namespace moe

// Internal services of moe_api.hip for the entry points defined in other files.
namespace moe {
// moe_ffn with ids/w given, its decode path (M <= MOE_DECODE_MAX_M) using hbuf
// (decode_scratch_floats(hidden, inter)) as its scratch.
moe_status ffn_with_scratch(const char *fn, moe_ctx *ctx, int layer, const float *x, const uint16_t *ids,
                            const float *w, int M, float *y, int flags, void *stream, float *hbuf);
int ctx_device(const moe_ctx *ctx);
// moe_ffn_noalloc's set-up on `device` (current): the device address of its static scratch,
// looked up once per device and kept.
hipError_t noalloc_prepare(int device);
int ctx_inter(const moe_ctx *ctx);
// Sets the calling thread's moe_last_error message and returns st.
moe_status set_error(moe_status st, const char *msg);
} // namespace moe
