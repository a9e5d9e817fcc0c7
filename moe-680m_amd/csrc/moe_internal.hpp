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

constexpr int PF_BM = 64; // prefill tile rows (token slots)

struct DecodeArgs {
    LayerPtrs L;
    const float *x;
    const uint16_t *ids;
    const float *w;
    float *y;
    float *hbuf;     // [M][9][I] f32
    uint32_t *flags; // sticky device flags
    int M, E, accumulate, rmsnorm;
    float c;
};

struct BucketArgs {
    const uint16_t *ids;
    const float *w;
    int M, E1; // E1 = n_experts + 1 buckets
    uint32_t *ranges;     // [E1+1]
    uint16_t *sorted_tok; // [9M]
    float *sorted_w;      // [9M]
    uint32_t *pos;        // [M][9] or null
    uint32_t *chunk_cnt;  // workspace [ceil(M/64)][E1]
    Tile *tiles;          // [tile_max] or null
    int tile_max, tile_bm;
    uint32_t *flags;
};

struct PrefillArgs {
    LayerPtrs L;
    const float *x;
    __bf16 *xb;          // [M][H] bf16 (normalised if requested)
    const uint16_t *sorted_tok;
    const float *sorted_w;
    const uint32_t *pos; // [M][9]
    const Tile *tiles;
    __bf16 *hs;          // [9M][I] bf16, sorted slot order
    float *part;         // [9M][H] f32, c*w-scaled expert outputs, sorted slot order
    float *y;
    int M, E, accumulate, rmsnorm, tile_max;
    float c;
};

hipError_t launch_dequant(const void *blocks, uint64_t n_sb, float *out, hipStream_t st);
hipError_t launch_gen_iq4xs(void *dst, uint64_t n, uint64_t seed, uint64_t first, hipStream_t st);
hipError_t launch_gen_normal(float *dst, uint64_t n, uint64_t seed, uint64_t first, float mean,
                             float stdv, hipStream_t st);
hipError_t launch_gen_logits(float *dst, int M, int E, uint64_t seed, int kind, double param,
                             double hot_value, hipStream_t st);
hipError_t launch_router_topk(const float *logits, int M, int E, int renorm, uint16_t *ids,
                              float *w, hipStream_t st);
hipError_t launch_bucket_fill(const BucketArgs &a, hipStream_t st);
hipError_t launch_decode(int H, int I, const DecodeArgs &a, hipStream_t st);
hipError_t launch_prefill(int H, int I, const PrefillArgs &a, hipStream_t st);

inline int tile_max_for(int M, int E1) { return (9 * M + PF_BM - 1) / PF_BM + E1; }

} // namespace moe
