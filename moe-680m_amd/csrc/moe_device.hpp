// moe_device.hpp -- device helpers shared by the gfx950 kernels of the MoE FFN path.
//
// IQ4_XS (ggml block_iq4_xs, 136 bytes per 256 weights):
//   u16 d (f16) @0 | u16 scales_h @2 | u8 scales_l[4] @4 | u8 qs[128] @8
//   sub-block ib (0..7) covers weights 32*ib .. 32*ib+31 with scale
//     dl = d * (ls - 32),  ls = (scales_l nibble ib) | (scales_h bits 2ib..2ib+1) << 4
//   byte j of qs[16*ib .. 16*ib+15] holds weight j in its low nibble and j+16 in its high
//   nibble; the value is dl * kvalues_iq4nl[nibble].
// It replaces the reference's 36-byte block decoder (shaders/common.glsl:61-86), which
// re-read d and both bit planes per weight through 8-bit word loads.  Here a lane owns one
// sub-block: the 8-byte header and the 16 qs bytes arrive as one 64-bit and one 128-bit
// load, the codebook lookup is three v_perm_b32 per four weights, and the scale is applied
// once per sub-block.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

constexpr int QK = 256;       // weights per super-block
constexpr int SB_BYTES = 136; // bytes per super-block
constexpr int TOPK = 8;
constexpr int SLOTS = 9;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// kvalues_iq4nl = {-127,-104,-83,-65,-49,-35,-22,-10,1,13,25,38,53,69,89,113},
// stored +128 as unsigned bytes (1..241) so v_cvt_f32_ubyte{0..3} converts them in one
// instruction; callers subtract 128 * sum(x) once per sub-block.
constexpr uint32_t KVB0 = 1u | (24u << 8) | (45u << 16) | (63u << 24);
constexpr uint32_t KVB1 = 79u | (93u << 8) | (106u << 16) | (118u << 24);
constexpr uint32_t KVB2 = 129u | (141u << 8) | (153u << 16) | (166u << 24);
constexpr uint32_t KVB3 = 181u | (197u << 8) | (217u << 16) | (241u << 24);
// The same codebook as two's-complement int8 bytes (exact small integers).
constexpr uint32_t KVS0 = 0x81u | (0x98u << 8) | (0xADu << 16) | (0xBFu << 24);
constexpr uint32_t KVS1 = 0xCFu | (0xDDu << 8) | (0xEAu << 16) | (0xF6u << 24);
constexpr uint32_t KVS2 = 0x01u | (0x0Du << 8) | (0x19u << 16) | (0x26u << 24);
constexpr uint32_t KVS3 = 0x35u | (0x45u << 8) | (0x59u << 16) | (0x71u << 24);

// Four nibble indices (bits 0..3 of each byte, upper bits ignored by the masks below)
// -> four table bytes.  v_perm_b32 picks bytes 0..7 of {S0:S1}; two perms cover table
// halves 0..7 and 8..15 and a third chooses per byte on index bit 3.
template <uint32_t T0, uint32_t T1, uint32_t T2, uint32_t T3>
__device__ __forceinline__ uint32_t lookup16(uint32_t idx_lo3, uint32_t sel_bit3) {
    uint32_t lo = __builtin_amdgcn_perm(T1, T0, idx_lo3);
    uint32_t hi = __builtin_amdgcn_perm(T3, T2, idx_lo3);
    return __builtin_amdgcn_perm(hi, lo, sel_bit3);
}

// qs dword q (4 bytes = weights j..j+3 low nibbles, j+16..j+19 high nibbles).
// Returns biased codebook bytes for the low nibbles (lo) and the high nibbles (hi).
__device__ __forceinline__ void kv_biased8(uint32_t q, uint32_t &lo, uint32_t &hi) {
    uint32_t a_lo = q & 0x07070707u;
    uint32_t s_lo = ((q >> 1) & 0x04040404u) | 0x03020100u;
    uint32_t a_hi = (q >> 4) & 0x07070707u;
    uint32_t s_hi = ((q >> 5) & 0x04040404u) | 0x03020100u;
    lo = lookup16<KVB0, KVB1, KVB2, KVB3>(a_lo, s_lo);
    hi = lookup16<KVB0, KVB1, KVB2, KVB3>(a_hi, s_hi);
}

__device__ __forceinline__ void kv_signed8(uint32_t q, uint32_t &lo, uint32_t &hi) {
    uint32_t a_lo = q & 0x07070707u;
    uint32_t s_lo = ((q >> 1) & 0x04040404u) | 0x03020100u;
    uint32_t a_hi = (q >> 4) & 0x07070707u;
    uint32_t s_hi = ((q >> 5) & 0x04040404u) | 0x03020100u;
    lo = lookup16<KVS0, KVS1, KVS2, KVS3>(a_lo, s_lo);
    hi = lookup16<KVS0, KVS1, KVS2, KVS3>(a_hi, s_hi);
}

__device__ __forceinline__ float ubyte(uint32_t v, int i) {
    return (float)((v >> (8 * i)) & 0xFFu); // v_cvt_f32_ubyte{i}
}
__device__ __forceinline__ float sbyte(uint32_t v, int i) {
    return (float)(int32_t)((int32_t)(v << (24 - 8 * i)) >> 24);
}

// Exact IEEE f16 -> f32 (v_cvt_f32_f16; f16 denormals are kept in the default FP mode).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu));
    return (float)v;
}

// Sub-block scale from the 8-byte header (hdr.x = d | scales_h << 16, hdr.y = scales_l).
__device__ __forceinline__ float sub_scale(u32x2 hdr, int ib) {
    float d = f16_bits_to_f32(hdr.x);
    uint32_t sh = hdr.x >> 16;
    int ls = (int)((hdr.y >> (4 * ib)) & 0xFu) | (int)(((sh >> (2 * ib)) & 3u) << 4);
    return d * (float)(ls - 32);
}

// 16 qs bytes of one sub-block against its 32 activations: sum_j kv[q_j] * x_j,
// returned unscaled (caller multiplies by dl).  xs = sum of the 32 activations.
__device__ __forceinline__ float subblock_dot(u32x4 qs, const float *xv, float xs) {
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        uint32_t lo, hi;
        kv_biased8(qs[w], lo, hi);
        a0 = __builtin_fmaf(ubyte(lo, 0), xv[4 * w + 0], a0);
        a1 = __builtin_fmaf(ubyte(lo, 1), xv[4 * w + 1], a1);
        a2 = __builtin_fmaf(ubyte(lo, 2), xv[4 * w + 2], a2);
        a3 = __builtin_fmaf(ubyte(lo, 3), xv[4 * w + 3], a3);
        a0 = __builtin_fmaf(ubyte(hi, 0), xv[16 + 4 * w + 0], a0);
        a1 = __builtin_fmaf(ubyte(hi, 1), xv[16 + 4 * w + 1], a1);
        a2 = __builtin_fmaf(ubyte(hi, 2), xv[16 + 4 * w + 2], a2);
        a3 = __builtin_fmaf(ubyte(hi, 3), xv[16 + 4 * w + 3], a3);
    }
    return ((a0 + a1) + (a2 + a3)) - 128.f * xs;
}

// ---------------------------------------------------------------- cross-lane sums
// DPP sums inside a row of 16 lanes; every lane of the row ends with the row total and
// every lane computes it in the same association, so the result is deterministic.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                  CTRL, 0xF, 0xF, true));
}

__device__ __forceinline__ float sum16(float v) {
    v += dpp_mov<0xB1>(v);  // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);  // quad_perm [2,3,0,1]
    v += dpp_mov<0x141>(v); // row_half_mirror
    v += dpp_mov<0x140>(v); // row_mirror
    return v;
}

// Sum over groups of G lanes (G in 8,16,32,64), result in every lane of the group.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(G == 8 || G == 16 || G == 32 || G == 64, "group size");
    if constexpr (G == 8) {
        v += dpp_mov<0xB1>(v);
        v += dpp_mov<0x4E>(v);
        v += dpp_mov<0x141>(v);
        return v;
    } else {
        v = sum16(v);
        if constexpr (G >= 32) v += __shfl_xor(v, 16);
        if constexpr (G == 64) v += __shfl_xor(v, 32);
        return v;
    }
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

// ---------------------------------------------------------------- expert table
struct LayerPtrs {
    const uint8_t *w1, *w3, *w2;
    uint64_t s1, s3, s2;
    const uint8_t *sw1, *sw3, *sw2;
};

__device__ __forceinline__ const uint8_t *expert_w(const uint8_t *base, uint64_t stride,
                                                   const uint8_t *shared, int e, int E) {
    return e == E ? shared : base + (uint64_t)e * stride;
}

template <typename T>
__device__ __forceinline__ T ldg(const void *p) {
    return *reinterpret_cast<const T *>(p);
}

__device__ __forceinline__ void set_flag(uint32_t *flags, uint32_t f) {
    if (flags) atomicOr(flags, f);
}

} // namespace moe
