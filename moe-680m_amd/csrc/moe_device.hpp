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
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Loads through the global address space: pointers read from memory (the layer table)
// are otherwise generic, and FLAT instructions also count against lgkmcnt, so every LDS
// wait would stall on outstanding weight loads.
#define MOE_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ T ldg(const void *p) {
    return *(const MOE_GLOBAL T *)p;
}

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
// (x & 0x04040404) | 0x03020100 in one v_bitop3_b32 (truth table 0xEA = (a & b) | c).
__device__ __forceinline__ uint32_t sel_bit3(uint32_t x) {
    return __builtin_amdgcn_bitop3_b32(x, 0x04040404u, 0x03020100u, 0xEA);
}

__device__ __forceinline__ void kv_biased8(uint32_t q, uint32_t &lo, uint32_t &hi) {
    uint32_t a_lo = q & 0x07070707u;
    uint32_t s_lo = sel_bit3(q >> 1);
    uint32_t a_hi = (q >> 4) & 0x07070707u;
    uint32_t s_hi = sel_bit3(q >> 5);
    lo = lookup16<KVB0, KVB1, KVB2, KVB3>(a_lo, s_lo);
    hi = lookup16<KVB0, KVB1, KVB2, KVB3>(a_hi, s_hi);
}

__device__ __forceinline__ void kv_signed8(uint32_t q, uint32_t &lo, uint32_t &hi) {
    uint32_t a_lo = q & 0x07070707u;
    uint32_t s_lo = sel_bit3(q >> 1);
    uint32_t a_hi = (q >> 4) & 0x07070707u;
    uint32_t s_hi = sel_bit3(q >> 5);
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

// ---------------------------------------------------------------- int8 activation planes
// The decode kernels read activations as two int8 planes per 32-element chunk c (one IQ4_XS
// sub-block of K):
//     x_i ~= s_c * (xh_i + xl_i / 256),  s_c = max_c |x| / 127,  xh = rint(x / s_c),
//     xl = rint(256 * (x / s_c - xh)),
// so a sub-block dot is two integer dot products of the signed codebook bytes
// (v_dot4_i32_i8) with f32 scaling once per sub-block.  Error per element <= s_c / 512,
// i.e. <= 1.6e-5 of the chunk's largest |x|.
__device__ __forceinline__ float quant_ratio(float am) { return am > 1e-30f ? 127.0f * __builtin_amdgcn_rcpf(am) : 0.0f; }

// LDS planes: chunk c at XQS * c: xh dwords 0..7 (elements 4d..4d+3), xl dwords 8..15,
// 4 pad dwords (a lane's 128-bit reads of its chunk are conflict-free across lanes).
constexpr int XQS = 20;

// Four consecutive activations (ratio r = 127 / chunk max) -> their xh and xl bytes.
__device__ __forceinline__ void quant4(f32x4 v, float r, uint32_t &h, uint32_t &l) {
    h = 0u;
    l = 0u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float u = v[i] * r;
        const float hi = fminf(fmaxf(rintf(u), -127.0f), 127.0f);
        const float lo = fminf(fmaxf(rintf((u - hi) * 256.0f), -127.0f), 127.0f);
        h |= ((uint32_t)(int)hi & 0xFFu) << (8 * i);
        l |= ((uint32_t)(int)lo & 0xFFu) << (8 * i);
    }
}

// One qs dword (weights 4d..4d+3 low nibbles, 16+4d.. high nibbles) against the planes'
// dwords of those elements: xh_lo = dword d, xh_hi = dword 4+d (and the same for xl).
// lo, hi: the signed codebook bytes of the dword's low and high nibbles (kv_signed8).
__device__ __forceinline__ void dword_idot(uint32_t lo, uint32_t hi, uint32_t xh_lo, uint32_t xh_hi, uint32_t xl_lo,
                                           uint32_t xl_hi, int &ah, int &al) {
    ah = __builtin_amdgcn_sdot4((int)lo, (int)xh_lo, ah, false);
    ah = __builtin_amdgcn_sdot4((int)hi, (int)xh_hi, ah, false);
    al = __builtin_amdgcn_sdot4((int)lo, (int)xl_lo, al, false);
    al = __builtin_amdgcn_sdot4((int)hi, (int)xl_hi, al, false);
}

// Whole sub-block, already looked up (kv[2d], kv[2d+1] = kv_signed8 of qs dword d), against
// chunk planes xh[8], xl[8]: sum kv * (xh + xl/256), unscaled.
__device__ __forceinline__ float subblock_idot(const uint32_t (&kv)[8], const uint32_t (&xh)[8],
                                               const uint32_t (&xl)[8]) {
    int ah = 0, al = 0;
#pragma unroll
    for (int d = 0; d < 4; ++d) dword_idot(kv[2 * d], kv[2 * d + 1], xh[d], xh[4 + d], xl[d], xl[4 + d], ah, al);
    return __builtin_fmaf((float)al, 1.0f / 256.0f, (float)ah);
}

// 8 weights of one qs dword -- weights 4d..4d+3 (low nibbles) and 16+4d..16+4d+3 (high
// nibbles) of a sub-block, as the biased codebook bytes lo, hi (kv_biased8) -- against their
// activations xl[0..3], xh[0..3]; unscaled.
__device__ __forceinline__ float dword_dot(uint32_t lo, uint32_t hi, const float *xl, const float *xh) {
    float a0 = ubyte(lo, 0) * xl[0], a1 = ubyte(lo, 1) * xl[1];
    a0 = __builtin_fmaf(ubyte(lo, 2), xl[2], a0);
    a1 = __builtin_fmaf(ubyte(lo, 3), xl[3], a1);
    a0 = __builtin_fmaf(ubyte(hi, 0), xh[0], a0);
    a1 = __builtin_fmaf(ubyte(hi, 1), xh[1], a1);
    a0 = __builtin_fmaf(ubyte(hi, 2), xh[2], a0);
    a1 = __builtin_fmaf(ubyte(hi, 3), xh[3], a1);
    const float xs = ((xl[0] + xl[1]) + (xl[2] + xl[3])) + ((xh[0] + xh[1]) + (xh[2] + xh[3]));
    return (a0 + a1) - 128.f * xs;
}

// Whole sub-block, already looked up (kv[2d], kv[2d+1] = kv_biased8 of qs dword d), against
// its 32 activations xv; xs = their sum.  Unscaled.
__device__ __forceinline__ float subblock_dot(const uint32_t (&kv)[8], const float (&xv)[32], float xs) {
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const uint32_t lo = kv[2 * d], hi = kv[2 * d + 1];
        a0 = __builtin_fmaf(ubyte(lo, 0), xv[4 * d + 0], a0);
        a1 = __builtin_fmaf(ubyte(lo, 1), xv[4 * d + 1], a1);
        a2 = __builtin_fmaf(ubyte(lo, 2), xv[4 * d + 2], a2);
        a3 = __builtin_fmaf(ubyte(lo, 3), xv[4 * d + 3], a3);
        a0 = __builtin_fmaf(ubyte(hi, 0), xv[16 + 4 * d + 0], a0);
        a1 = __builtin_fmaf(ubyte(hi, 1), xv[16 + 4 * d + 1], a1);
        a2 = __builtin_fmaf(ubyte(hi, 2), xv[16 + 4 * d + 2], a2);
        a3 = __builtin_fmaf(ubyte(hi, 3), xv[16 + 4 * d + 3], a3);
    }
    return ((a0 + a1) + (a2 + a3)) - 128.f * xs;
}

// Biased codebook bytes b = kv + 128 (a kv_biased8 word, 4 weights) as two words of f16
// pairs 1024 + b: exponent byte 0x64 over each byte (exact; b < 1024).
__device__ __forceinline__ void kv_magic_f16(uint32_t bytes, uint32_t &p01, uint32_t &p23) {
    p01 = __builtin_amdgcn_perm(0x64646464u, bytes, 0x04010400u);
    p23 = __builtin_amdgcn_perm(0x64646464u, bytes, 0x04030402u);
}

// acc + w * x, w the low or high f16 half of a word, x and acc f32: one v_fma_mix_f32 (the
// f16 widened exactly, one rounding) -- what fmaf((float)w, x, acc) computes, in one
// instruction where the compiler emits a conversion and an FMA.
__device__ __forceinline__ float fma_mix_lo(uint32_t w, float x, float acc) {
    float d;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(d) : "v"(w), "v"(x), "v"(acc));
    return d;
}
__device__ __forceinline__ float fma_mix_hi(uint32_t w, float x, float acc) {
    float d;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(d) : "v"(w), "v"(x), "v"(acc));
    return d;
}

// subblock_dot from the same kv_biased8 words, each as f16 pairs 1024 + b: one
// v_fma_mix_f32 per weight instead of a byte conversion and an FMA; the offset 1024 + 128
// comes off once, with the activations' sum xs.  Unscaled.
__device__ __forceinline__ float subblock_dot_mix(const uint32_t (&kv)[8], const float (&xv)[32], float xs) {
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        uint32_t l01, l23, h01, h23;
        kv_magic_f16(kv[2 * d], l01, l23);
        kv_magic_f16(kv[2 * d + 1], h01, h23);
        a0 = fma_mix_lo(l01, xv[4 * d + 0], a0);
        a1 = fma_mix_hi(l01, xv[4 * d + 1], a1);
        a2 = fma_mix_lo(l23, xv[4 * d + 2], a2);
        a3 = fma_mix_hi(l23, xv[4 * d + 3], a3);
        a0 = fma_mix_lo(h01, xv[16 + 4 * d + 0], a0);
        a1 = fma_mix_hi(h01, xv[16 + 4 * d + 1], a1);
        a2 = fma_mix_lo(h23, xv[16 + 4 * d + 2], a2);
        a3 = fma_mix_hi(h23, xv[16 + 4 * d + 3], a3);
    }
    return ((a0 + a1) + (a2 + a3)) - 1152.f * xs;
}

// ---------------------------------------------------------------- split weight layout
// The library's one resident copy of every bound matrix (k_repack_split): for a matrix of
// `rows` rows of SBR super-blocks each,
//     [rows * SBR qs blocks of 128 bytes, row-major] [rows * SBR headers of 8 bytes, same order]
// -- the bytes of the GGML layout (136 per super-block) split in two, so that every 16-byte
// qs read is aligned and a row's headers are 8*SBR contiguous bytes.
template <int SBR>
__device__ __forceinline__ uint32_t split_qs(int row, int sb) { return (uint32_t)((row * SBR + sb) * 128); }
template <int ROWS, int SBR>
__device__ __forceinline__ uint32_t split_hdr(int row, int sb) {
    return (uint32_t)(ROWS * SBR * 128 + (row * SBR + sb) * 8);
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

// Whole-wave sum as a wave-uniform value: row sums by DPP, then the four row totals read
// with v_readlane and added in a fixed order (no LDS round trip).
__device__ __forceinline__ float wave_sum(float v) {
    v = sum16(v);
    const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (a + b) + (c + d);
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, dpp_u32<0xB1>(v));
    v = max(v, dpp_u32<0x4E>(v));
    v = max(v, dpp_u32<0x141>(v));
    v = max(v, dpp_u32<0x140>(v));
    const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
    const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
    const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
    const uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
    return max(max(a, b), max(c, d));
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
    v = min(v, dpp_u32<0xB1>(v));
    v = min(v, dpp_u32<0x4E>(v));
    v = min(v, dpp_u32<0x141>(v));
    v = min(v, dpp_u32<0x140>(v));
    const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
    const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
    const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
    const uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
    return min(min(a, b), min(c, d));
}

// Max over the wave, complete in lane 63 only: row maxima by DPP, then row_bcast:15 (rows
// 1, 3 take the last lane of the row below) and row_bcast:31 (rows 2, 3 take lane 31), read
// from lane 63 -- one readlane instead of four on the dependency chain.  The DPP source
// defaults to 0, the identity of an unsigned max (rows outside a row mask), which lets
// each step compile to one v_max_u32 with a DPP operand.
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_max_step(uint32_t v) {
    return max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWS, 0xF, false));
}
__device__ __forceinline__ uint32_t wave_max_last_u32(uint32_t v) {
    v = dpp_max_step<0xB1, 0xF>(v);  // quad_perm [1,0,3,2]
    v = dpp_max_step<0x4E, 0xF>(v);  // quad_perm [2,3,0,1]
    v = dpp_max_step<0x141, 0xF>(v); // row_half_mirror
    v = dpp_max_step<0x140, 0xF>(v); // row_mirror
    v = dpp_max_step<0x142, 0xA>(v); // row_bcast:15
    v = dpp_max_step<0x143, 0xC>(v); // row_bcast:31
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
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

// Whole-wave sum that is complete in lane 63 only (lanes of rows 0-2 hold partial sums):
// row sums by DPP, then row_bcast:15 (rows 1, 3 += last lane of the row below) and
// row_bcast:31 (rows 2, 3 += lane 31).  Six DPP adds, no readlane.
__device__ __forceinline__ float wave_sum_last(float v) {
    v = sum16(v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142, 0xA, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143, 0xC, 0xF, false));
    return v;
}

// Total of each group of G lanes, complete in lane 63 for G = 64 (DPP only, no readlane on
// the dependency chain) and in every lane otherwise.
template <int G>
__device__ __forceinline__ float row_total(float v) {
    if constexpr (G == 64) return wave_sum_last(v);
    else return group_sum<G>(v);
}
// The lane of a G-lane group that holds row_total's result.
template <int G>
constexpr int row_total_lane() { return G == 64 ? 63 : 0; }

// Total over each group of G lanes (G = 64: wave-uniform value through readlane).
template <int G>
__device__ __forceinline__ float lanes_total(float v) {
    if constexpr (G == 64) return wave_sum(v);
    else return group_sum<G>(v);
}

// 32 consecutive f32 (16-byte aligned) into registers as eight 128-bit loads.
__device__ __forceinline__ void load32(const float *__restrict__ src, float (&v)[32]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        f32x4 q = ldg<f32x4>(src + 4 * i);
        v[4 * i + 0] = q[0];
        v[4 * i + 1] = q[1];
        v[4 * i + 2] = q[2];
        v[4 * i + 3] = q[3];
    }
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }
// The same with v_rcp_f32 (1 ulp) in place of the IEEE division sequence.
__device__ __forceinline__ float silu_rcp(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

// Workgroup barrier for LDS traffic only.  __syncthreads() also waits for every global
// load the wave has in flight (the barrier's release fence needs vmcnt(0)), which would
// stall on weight loads issued ahead of use.  Use it where the workgroup exchanges data
// through LDS only.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// ---------------------------------------------------------------- router (one wave)
__device__ __forceinline__ float router_key(float v) {
    if (v != v) v = -INFINITY; // NaN never wins and weighs 0 unless every logit is -inf/NaN
    if (v == 0.0f) v = 0.0f;   // -0 ties with +0
    return v;
}
__device__ __forceinline__ uint32_t ord32(float v) {
    uint32_t b = __builtin_bit_cast(uint32_t, v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float unord32(uint32_t o) {
    uint32_t b = (o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o;
    return __builtin_bit_cast(float, b);
}

// A token's E logits, lane + 64j into v[j]: unconditional in-bounds loads (index clamped,
// the surplus masked later), so all NV are in flight together.
template <int NV>
__device__ __forceinline__ void load_logits(const float *__restrict__ l, int E, int lane, float (&v)[NV]) {
#pragma unroll
    for (int j = 0; j < NV; ++j) v[j] = ldg<float>(l + min(lane + 64 * j, E - 1));
}

// Softmax + top-8 of one token's E logits (8 <= E <= 64*NV) by the calling wave, from the
// values load_logits returned.  Lane r < 8 comes out with rank r -- ids by (logit desc,
// index asc) -- and its weight (softmax probability, or renormalised over the 8 when
// renorm); lane 8 and above with the shared expert (id E, weight 1).
// A round: each lane's best remaining key, its wave max in lane 63, a ballot of the lanes
// holding it.  One lane: it wins with its lowest such index.  An exact tie across lanes:
// the smallest index among the holders, by a min reduction.  The sums keep one order --
// Z = (...(z_0 + z_1) + ...) + z_{NV-1}, z_j the wave_sum of the terms of logits 64j..64j+63;
// the top-8 sum over ranks 0..7 -- which route_wg4 keeps too, so every routing site agrees bit
// for bit.
template <int NV>
__device__ __forceinline__ void route_values_exact(const float (&raw)[NV], int E, int renorm, int lane, int &id,
                                                   float &wt) {
    float kf[NV], ex[NV];
    uint32_t ord[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int i = lane + 64 * j;
        kf[j] = (i < E) ? router_key(raw[j]) : -INFINITY;
        ord[j] = (i < E) ? ord32(kf[j]) : 0u; // 0 sorts below every real key (-inf is 0x007FFFFF)
    }
    float s8 = 0.f, my_e = 1.0f;
    int my_id = E;
#pragma unroll
    for (int r = 0; r < TOPK; ++r) {
        uint32_t kb = ord[0];
#pragma unroll
        for (int j = 1; j < NV; ++j) kb = max(kb, ord[j]);
        const uint32_t K = wave_max_last_u32(kb);
        if (r == 0) {
            const float m = unord32(K);
#pragma unroll
            for (int j = 0; j < NV; ++j)
                ex[j] = (lane + 64 * j < E) ? ((kf[j] == m) ? 1.0f : expf(kf[j] - m)) : 0.0f;
        }
        int jl = 0; // the lane's lowest j holding K (when it holds K)
        float el = ex[0];
#pragma unroll
        for (int j = NV - 1; j >= 0; --j)
            if (ord[j] == K) {
                jl = j;
                el = ex[j];
            }
        const uint64_t hit = __ballot(kb == K);
        int w = (int)__builtin_ctzll(hit);
        if (__builtin_popcountll(hit) > 1)
            w = (int)(wave_min_u32(kb == K ? (uint32_t)(lane + 64 * jl) : 0xFFFFFFFFu) & 63u);
        const int jw = __builtin_amdgcn_readlane(jl, w);
        const float e = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, el), w));
#pragma unroll
        for (int j = 0; j < NV; ++j)
            if (lane == w && j == jw) ord[j] = 0u;
        s8 += e;
        if (lane == r) {
            my_id = w + 64 * jw;
            my_e = e;
        }
    }
    float Z = wave_sum(ex[0]);
#pragma unroll
    for (int j = 1; j < NV; ++j) Z += wave_sum(ex[j]);
    id = my_id;
    wt = (lane < TOPK) ? my_e / (renorm ? s8 : Z) : 1.0f;
}

// The same routing, faster where no two of the winning keys tie (the common case), and
// bit for bit equal to route_values_exact: each lane sorts its NV keys once (key desc, j asc), a
// round is then the wave max of the lanes' first keys and a shift on the lanes holding it, with
// nothing else on the rounds' dependency chain -- the round's ballot, the winner's index and
// softmax term are kept and read after the rounds.  A round whose key several lanes hold (a
// tie, where the exact rule picks the lowest index among them) sends the call to
// route_values_exact, from the start.
template <int NV>
__device__ __forceinline__ void route_values(const float (&raw)[NV], int E, int renorm, int lane, int &id,
                                             float &wt) {
    float kf[NV], ex[NV], es[NV];
    uint32_t key[NV], js[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int i = lane + 64 * j;
        kf[j] = (i < E) ? router_key(raw[j]) : -INFINITY;
        key[j] = (i < E) ? ord32(kf[j]) : 0u; // 0 sorts below every real key (-inf is 0x007FFFFF)
        js[j] = (uint32_t)j;
    }
    uint32_t k0 = key[0];
#pragma unroll
    for (int j = 1; j < NV; ++j) k0 = max(k0, key[j]);
    const uint32_t K0 = wave_max_last_u32(k0);
    const float m = unord32(K0);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        ex[j] = (lane + 64 * j < E) ? ((kf[j] == m) ? 1.0f : expf(kf[j] - m)) : 0.0f;
        es[j] = ex[j];
    }
    // insertion sort: strictly greater keys move up, so equal keys keep ascending j
#pragma unroll
    for (int a = 1; a < NV; ++a)
#pragma unroll
        for (int b = a; b > 0; --b) {
            const bool sw = key[b] > key[b - 1];
            const uint32_t ka = key[b - 1], kb = key[b], ja = js[b - 1], jb = js[b];
            const float ea = es[b - 1], eb = es[b];
            key[b - 1] = sw ? kb : ka;
            key[b] = sw ? ka : kb;
            js[b - 1] = sw ? jb : ja;
            js[b] = sw ? ja : jb;
            es[b - 1] = sw ? eb : ea;
            es[b] = sw ? ea : eb;
        }
    uint64_t hit[TOPK];
    uint32_t ri[TOPK];
    float re[TOPK];
#pragma unroll
    for (int r = 0; r < TOPK; ++r) {
        const uint32_t K = r == 0 ? K0 : wave_max_last_u32(key[0]);
        const bool eq = key[0] == K;
        hit[r] = __ballot(eq);
        ri[r] = eq ? (uint32_t)(lane + 64 * (int)js[0]) : 0u;
        re[r] = eq ? es[0] : 0.0f;
#pragma unroll
        for (int p = 0; p < NV - 1; ++p) {
            key[p] = eq ? key[p + 1] : key[p];
            js[p] = eq ? js[p + 1] : js[p];
            es[p] = eq ? es[p + 1] : es[p];
        }
        key[NV - 1] = eq ? 0u : key[NV - 1];
    }
    bool tie = false;
#pragma unroll
    for (int r = 0; r < TOPK; ++r) tie = tie || __builtin_popcountll(hit[r]) != 1;
    if (tie) {
        route_values_exact<NV>(raw, E, renorm, lane, id, wt);
        return;
    }
    float s8 = 0.f, my_e = 1.0f;
    int my_id = E;
#pragma unroll
    for (int r = 0; r < TOPK; ++r) {
        const int w = (int)__builtin_ctzll(hit[r]);
        const int ir = __builtin_amdgcn_readlane((int)ri[r], w);
        const float e = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, re[r]), w));
        s8 += e;
        if (lane == r) {
            my_id = ir;
            my_e = e;
        }
    }
    float Z = wave_sum(ex[0]);
#pragma unroll
    for (int j = 1; j < NV; ++j) Z += wave_sum(ex[j]);
    id = my_id;
    wt = (lane < TOPK) ? my_e / (renorm ? s8 : Z) : 1.0f;
}

template <int NV>
__device__ __forceinline__ void route_wave(const float *__restrict__ l, int E, int renorm, int lane, int &id,
                                           float &wt) {
    float raw[NV];
    load_logits<NV>(l, E, lane, raw);
    route_values<NV>(raw, E, renorm, lane, id, wt);
}

// The same routing by the four waves of a workgroup, wave w taking logits 64w..64w+63, one per
// lane; every wave ends as route_values ends (lane r < 8: rank r and its weight; lane 8 and
// above: the shared expert), with bit-identical ids and weights.  Each wave ranks its own
// logits (a round: one wave max, a ballot, the winner's lane cleared -- the lowest lane holding the max is
// the lowest index), then every wave merges the 32 candidates from LDS, wave-major, so lane
// order is index order among equal keys.  Two LDS-only barriers; all 256 threads must call it.
struct RouteLds {
    uint32_t key[4][TOPK], idx[4][TOPK];
    float z[4];
};
// raw: logit 64 * wv + lane, already loaded (any value past E).
__device__ __forceinline__ void route_wg4v(float raw, int E, int renorm, int lane, int wv, RouteLds &R, int &id,
                                           float &wt) {
    const int i = 64 * wv + lane;
    const float kf = (i < E) ? router_key(raw) : -INFINITY;
    uint32_t o = (i < E) ? ord32(kf) : 0u; // 0 sorts below every real key
    uint32_t mk = 0u, mi = 0u;
#pragma unroll
    for (int r = 0; r < TOPK; ++r) {
        const uint32_t K = wave_max_last_u32(o);
        const int w = (int)__builtin_ctzll(__ballot(o == K));
        o = lane == w ? 0u : o;
        if (lane == r) {
            mk = K;
            mi = (uint32_t)(64 * wv + w);
        }
    }
    if (lane < TOPK) {
        R.key[wv][lane] = mk;
        R.idx[wv][lane] = mi;
    }
    lds_barrier();
    uint32_t c = lane < 4 * TOPK ? R.key[lane / TOPK][lane % TOPK] : 0u;
    const uint32_t ci = lane < 4 * TOPK ? R.idx[lane / TOPK][lane % TOPK] : 0u;
    // the global max, then this wave's part of the softmax sum
    const float m = unord32(wave_max_last_u32(c));
    const float zw = wave_sum((i < E) ? ((kf == m) ? 1.0f : expf(kf - m)) : 0.0f);
    if (lane == 0) R.z[wv] = zw;
    int my_id = E;
    uint32_t my_k = 0u;
#pragma unroll
    for (int r = 0; r < TOPK; ++r) {
        const uint32_t K = wave_max_last_u32(c);
        const int w = (int)__builtin_ctzll(__ballot(c == K));
        const int idx = __builtin_amdgcn_readlane((int)ci, w);
        c = lane == w ? 0u : c;
        if (lane == r) {
            my_id = idx;
            my_k = K;
        }
    }
    lds_barrier();
    const float Z = ((R.z[0] + R.z[1]) + R.z[2]) + R.z[3];
    const float kr = unord32(my_k);
    const float e = (lane < TOPK) ? ((kr == m) ? 1.0f : expf(kr - m)) : 1.0f;
    float s8 = 0.f;
#pragma unroll
    for (int r = 0; r < TOPK; ++r) s8 += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e), r));
    id = my_id;
    wt = (lane < TOPK) ? e / (renorm ? s8 : Z) : 1.0f;
}
__device__ __forceinline__ void route_wg4(const float *__restrict__ l, int E, int renorm, int lane, int wv,
                                          RouteLds &R, int &id, float &wt) {
    route_wg4v(ldg<float>(l + min(64 * wv + lane, E - 1)), E, renorm, lane, wv, R, id, wt);
}

// ---------------------------------------------------------------- expert table
struct LayerPtrs {
    const uint8_t *w1, *w3, *w2;
    uint64_t s1, s3, s2;
    const uint8_t *sw1, *sw3, *sw2;
};

// A LayerPtrs entry of a device table, read field by field through global loads.
__device__ __forceinline__ LayerPtrs load_layer(const LayerPtrs *p) {
    const uint64_t *q = reinterpret_cast<const uint64_t *>(p);
    LayerPtrs L;
    L.w1 = (const uint8_t *)ldg<uint64_t>(q + 0);
    L.w3 = (const uint8_t *)ldg<uint64_t>(q + 1);
    L.w2 = (const uint8_t *)ldg<uint64_t>(q + 2);
    L.s1 = ldg<uint64_t>(q + 3);
    L.s3 = ldg<uint64_t>(q + 4);
    L.s2 = ldg<uint64_t>(q + 5);
    L.sw1 = (const uint8_t *)ldg<uint64_t>(q + 6);
    L.sw3 = (const uint8_t *)ldg<uint64_t>(q + 7);
    L.sw2 = (const uint8_t *)ldg<uint64_t>(q + 8);
    return L;
}
static_assert(sizeof(LayerPtrs) == 72, "LayerPtrs is nine 8-byte fields");

__device__ __forceinline__ const uint8_t *expert_w(const uint8_t *base, uint64_t stride,
                                                   const uint8_t *shared, int e, int E) {
    return e == E ? shared : base + (uint64_t)e * stride;
}


// ---------------------------------------------------------------- cross-XCD exchange
// Each XCD has its own L2.  A word published for workgroups on other XCDs is stored at agent
// scope, which writes through the producer's L2; consumers read it with system-scope loads,
// which miss their own L2 and see memory.  The buffer starts zeroed and a published f32
// carries its mantissa LSB forced to 1 (<= 1 ulp), so "LSB set" marks a written word.
__device__ __forceinline__ void tag_store(uint32_t *p, float v) {
    __hip_atomic_store((MOE_GLOBAL uint32_t *)p, __builtin_bit_cast(uint32_t, v) | 1u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
// 16 bytes as two relaxed 8-byte system-scope atomic loads (atomic, so a poll loop re-issues
// them every round; relaxed, so the compiler does not wait for each one).
__device__ __forceinline__ u32x4 remote_quad(const u32x4 *p) {
    const MOE_GLOBAL uint64_t *g = (const MOE_GLOBAL uint64_t *)p;
    const uint64_t lo = __hip_atomic_load(g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    const uint64_t hi = __hip_atomic_load(g + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    return u32x4{(uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32)};
}
__device__ __forceinline__ uint32_t quad_tagged(u32x4 v) { return v[0] & v[1] & v[2] & v[3] & 1u; }

__device__ __forceinline__ void set_flag(uint32_t *flags, uint32_t f) {
    if (flags) __hip_atomic_fetch_or((MOE_GLOBAL uint32_t *)flags, f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

} // namespace moe
