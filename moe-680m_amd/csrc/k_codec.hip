// k_codec.hip -- IQ4_XS decode test hook and the seeded input generators.
#include "moe_internal.hpp"

namespace moe {

// One thread per (super-block, sub-block): 8-byte header + 16 qs bytes -> 32 exact f32.
// Values are dl * kv with dl = d*(ls-32); both products are exact in f32 (at most 23
// significant bits), so the result is bit-identical to any correct decoder.
__global__ __launch_bounds__(256) void k_dequant_iq4xs(const uint8_t *__restrict__ blocks,
                                                       uint64_t n_sb, float *__restrict__ out) {
    uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= n_sb * 8) return;
    uint64_t sb = gid >> 3;
    int ib = (int)(gid & 7);
    const uint8_t *p = blocks + sb * SB_BYTES;
    u32x2 hdr = ldg<u32x2>(p);
    u32x4 qs;
#pragma unroll
    for (int w = 0; w < 4; ++w) qs[w] = ldg<uint32_t>(p + 8 + 16 * ib + 4 * w);
    float dl = sub_scale(hdr, ib);
    float *o = out + sb * QK + 32 * ib;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        uint32_t lo, hi;
        kv_signed8(qs[w], lo, hi);
        f32x4 vlo, vhi;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            vlo[i] = dl * sbyte(lo, i);
            vhi[i] = dl * sbyte(hi, i);
        }
        *reinterpret_cast<f32x4 *>(o + 4 * w) = vlo;
        *reinterpret_cast<f32x4 *>(o + 16 + 4 * w) = vhi;
    }
}

// ---------------------------------------------------------------- generator
// Counter-based: value i of stream `seed` is a function of (seed, i) only.
//   mix64      = splitmix64 finaliser (with its golden-ratio increment)
//   rng(s, i)  = mix64(s ^ mix64(i))
//   normal(i)  = Box-Muller on rng(s, 2i), rng(s, 2i+1), with log and cos(2 pi u) evaluated
//                by fixed series using IEEE basic operations only (no contraction), so the
//                same bits come out on any IEEE machine.
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__device__ __forceinline__ uint64_t rng(uint64_t seed, uint64_t i) { return mix64(seed ^ mix64(i)); }

__device__ double gen_log(double x) {
#pragma clang fp contract(off)
    int e;
    double m = frexp(x, &e);
    if (m < 0.70710678118654752440) {
        m = m * 2.0;
        e -= 1;
    }
    double s = (m - 1.0) / (m + 1.0);
    double s2 = s * s;
    double p = 1.0 / 23.0;
    for (int k = 21; k >= 1; k -= 2) {
        p = p * s2;
        p = p + 1.0 / (double)k;
    }
    double lm = 2.0 * s * p;
    double el = (double)e * 0.69314718055994530942;
    return el + lm;
}

__device__ double series_sin(double a) {
#pragma clang fp contract(off)
    double a2 = a * a, term = a, sum = a;
    for (int k = 1; k <= 11; ++k) {
        term = -term * a2 / (double)((2 * k) * (2 * k + 1));
        sum = sum + term;
    }
    return sum;
}
__device__ double series_cos(double a) {
#pragma clang fp contract(off)
    double a2 = a * a, term = 1.0, sum = 1.0;
    for (int k = 1; k <= 11; ++k) {
        term = -term * a2 / (double)((2 * k - 1) * (2 * k));
        sum = sum + term;
    }
    return sum;
}
__device__ double gen_cos2pi(double u) {
#pragma clang fp contract(off)
    double wv = u - floor(u + 0.5);
    wv = fabs(wv);
    double sgn = 1.0;
    if (wv > 0.25) {
        wv = 0.5 - wv;
        sgn = -1.0;
    }
    const double TWO_PI = 6.283185307179586476925;
    double r = (wv > 0.125) ? series_sin(TWO_PI * (0.25 - wv)) : series_cos(TWO_PI * wv);
    return sgn * r;
}
__device__ double box_muller(uint64_t r1, uint64_t r2) {
#pragma clang fp contract(off)
    double u1 = (double)((r1 >> 11) + 1) * 0x1.0p-53;
    double u2 = (double)(r2 >> 11) * 0x1.0p-53;
    double l = gen_log(u1);
    return sqrt(-2.0 * l) * gen_cos2pi(u2);
}

// f32 -> f16 bits, round to nearest even, in integer arithmetic.
__device__ uint32_t f32_to_f16_rne(float f) {
    uint32_t x = __builtin_bit_cast(uint32_t, f);
    uint32_t sign = (x >> 16) & 0x8000u, ex = (x >> 23) & 0xFFu, man = x & 0x7FFFFFu;
    if (ex == 0xFF) return sign | 0x7C00u | (man ? 0x200u : 0u);
    int e = (int)ex - 127 + 15;
    if (e >= 31) return sign | 0x7C00u;
    if (e <= 0) {
        if (e < -10) return sign;
        uint32_t m = man | 0x800000u;
        int shift = 14 - e;
        uint32_t q = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return sign | q;
    }
    uint32_t q = ((uint32_t)e << 10) | (man >> 13), rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return sign | q;
}

// Super-block b: qs bytes from rng(seed, 32b + 0..15), eight 6-bit scales from
// rng(seed, 32b + 16), d = f16(f32(|N(0,1)| * 2e-3)) from rng(seed, 32b + 17/18).
__global__ __launch_bounds__(256) void k_gen_iq4xs(uint8_t *__restrict__ dst, uint64_t n,
                                                   uint64_t seed, uint64_t first) {
    uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint64_t b = first + i;
    uint8_t *p = dst + i * SB_BYTES;
    for (int j = 0; j < 16; ++j) {
        uint64_t r = rng(seed, 32 * b + (uint64_t)j);
        *reinterpret_cast<u32x2 *>(p + 8 + 8 * j) = u32x2{(uint32_t)r, (uint32_t)(r >> 32)};
    }
    uint64_t rs = rng(seed, 32 * b + 16);
    uint32_t sh = 0, sl = 0;
    for (int ib = 0; ib < 8; ++ib) {
        uint32_t ls = (uint32_t)(rs >> (6 * ib)) & 63u;
        sl |= (ls & 15u) << (4 * ib);
        sh |= (ls >> 4) << (2 * ib);
    }
    double z = box_muller(rng(seed, 32 * b + 17), rng(seed, 32 * b + 18));
    double dv = fabs(z) * 2e-3;
    uint32_t dh = f32_to_f16_rne((float)dv);
    *reinterpret_cast<u32x2 *>(p) = u32x2{dh | (sh << 16), sl};
}

__global__ __launch_bounds__(256) void k_gen_normal(float *__restrict__ dst, uint64_t n,
                                                    uint64_t seed, uint64_t first, float mean,
                                                    float stdv) {
#pragma clang fp contract(off)
    uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint64_t k = first + i;
    double z = box_muller(rng(seed, 2 * k), rng(seed, 2 * k + 1));
    double v = z * (double)stdv;
    v = v + (double)mean;
    dst[i] = (float)v;
}

constexpr uint64_t TAG_PERM = 0x5045524Dull, TAG_HOTE = 0x484F5445ull, TAG_HOTT = 0x484F5454ull;

// Logits [M][E]: N(0,1) (element t*E+e of stream seed) + bias.  Zipf: bias_e =
// -s*log(rank_e), rank from sorting rng(seed^PERM, e); hot: token t is hot when
// u01(rng(seed^HOTT, t)) < p, and then its logit for expert rng(seed^HOTE, 0) % E is set.
__global__ __launch_bounds__(256) void k_gen_logits(float *__restrict__ dst, int M, int E,
                                                    uint64_t seed, int kind, double param,
                                                    double hot_value) {
#pragma clang fp contract(off)
    uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (uint64_t)M * (uint64_t)E) return;
    int t = (int)(gid / (uint64_t)E), e = (int)(gid % (uint64_t)E);
    double bias = 0.0;
    if (kind == 1) {
        uint64_t ke = rng(seed ^ TAG_PERM, (uint64_t)e);
        int rank = 1;
        for (int j = 0; j < E; ++j) {
            uint64_t kj = rng(seed ^ TAG_PERM, (uint64_t)j);
            rank += (kj < ke || (kj == ke && j < e)) ? 1 : 0;
        }
        double lr = gen_log((double)rank);
        bias = -param * lr;
    }
    double z = box_muller(rng(seed, 2 * gid), rng(seed, 2 * gid + 1));
    double v = z + bias;
    if (kind == 2) {
        double u = (double)(rng(seed ^ TAG_HOTT, (uint64_t)t) >> 11) * 0x1.0p-53;
        int hot = (int)(rng(seed ^ TAG_HOTE, 0) % (uint64_t)E);
        if (u < param && e == hot) v = hot_value;
    }
    dst[gid] = (float)v;
}

// ---------------------------------------------------------------- launchers
// ---------------------------------------------------------------- split repack
// One-time copy of a bound layer into the layout every kernel family reads.  Per matrix of nsb
// super-blocks (row-major: rows x super-blocks per row):
//     [nsb x 128-byte qs] [nsb x 8-byte header (d, scales_h, scales_l)]
// -- the bytes of the natural layout (136 per super-block) split in two, so that every
// 16-byte qs read is aligned and the headers a wave needs lie in a few cache lines.
__global__ __launch_bounds__(256) void k_repack_split(const uint8_t *__restrict__ src, uint64_t src_stride,
                                                      const uint8_t *__restrict__ shared, uint8_t *__restrict__ dst,
                                                      uint64_t dst_stride, int E, uint64_t nsb) {
    const int e = blockIdx.y;
    const uint8_t *m = (e == E) ? shared : src + (uint64_t)e * src_stride;
    uint8_t *o = dst + (uint64_t)e * dst_stride;
    // one thread per 8-byte word (17 per super-block; word 0 is the header)
    for (uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; t < nsb * 17;
         t += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t sb = t / 17;
        const int wd = (int)(t % 17);
        const uint64_t v = *reinterpret_cast<const uint64_t *>(m + sb * SB_BYTES + 8u * wd);
        uint8_t *to = wd == 0 ? o + nsb * 128 + sb * 8 : o + sb * 128 + 8u * (wd - 1);
        *reinterpret_cast<uint64_t *>(to) = v;
    }
}

hipError_t launch_repack_split(const void *src, uint64_t src_stride, const void *shared, void *dst,
                               uint64_t dst_stride, int E, int rows, int cols, hipStream_t st) {
    const uint64_t nsb = (uint64_t)rows * (cols / QK);
    const uint64_t blocks = (nsb * 17 + 255) / 256;
    dim3 grid((unsigned)(blocks < 4096 ? blocks : 4096), (unsigned)(E + 1));
    hipLaunchKernelGGL(k_repack_split, grid, dim3(256), 0, st, (const uint8_t *)src, src_stride,
                       (const uint8_t *)shared, (uint8_t *)dst, dst_stride, E, nsb);
    return hipGetLastError();
}

// One workgroup: thread 0 swaps the flags out; after an expired decode-stack wait, thread 0
// clears the abort word and all threads zero the stack's control words and exchange sets (an error path: its speed does not
// matter, and the usual call only reads and clears one word).
__global__ __launch_bounds__(1024) void k_flags_take(uint32_t *flags, uint32_t *dst, u32x4 *stack,
                                                     uint64_t stack_quads) {
    __shared__ uint32_t s_v;
    if (threadIdx.x == 0) {
        const uint32_t v =
            __hip_atomic_exchange((MOE_GLOBAL uint32_t *)flags, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *dst = v;
        s_v = v;
    }
    __syncthreads();
    // the abort word (flags[1]) goes too: the control words restart the epoch at 0, and an
    // abort tag left from a launch at epoch 0 would otherwise match the next epoch-0 launch
    if ((s_v & MOE_DEVFLAG_TIMEOUT) && threadIdx.x == 0)
        __hip_atomic_store((MOE_GLOBAL uint32_t *)(flags + 1), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (s_v & MOE_DEVFLAG_TIMEOUT)
        for (uint64_t q = threadIdx.x; q < stack_quads; q += blockDim.x)
            *(MOE_GLOBAL u32x4 *)(stack + q) = u32x4{0u, 0u, 0u, 0u};
}

hipError_t launch_flags_take(uint32_t *flags, uint32_t *dst, uint32_t *stack, size_t stack_words, hipStream_t st) {
    hipLaunchKernelGGL(k_flags_take, dim3(1), dim3(1024), 0, st, flags, dst, reinterpret_cast<u32x4 *>(stack),
                       (uint64_t)(stack_words / 4));
    return hipGetLastError();
}

hipError_t launch_dequant(const void *blocks, uint64_t n_sb, float *out, hipStream_t st) {
    uint64_t threads = n_sb * 8;
    if (threads == 0) return hipSuccess;
    dim3 grid((unsigned)((threads + 255) / 256));
    hipLaunchKernelGGL(k_dequant_iq4xs, grid, dim3(256), 0, st, (const uint8_t *)blocks, n_sb, out);
    return hipGetLastError();
}

hipError_t launch_gen_iq4xs(void *dst, uint64_t n, uint64_t seed, uint64_t first, hipStream_t st) {
    if (n == 0) return hipSuccess;
    dim3 grid((unsigned)((n + 255) / 256));
    hipLaunchKernelGGL(k_gen_iq4xs, grid, dim3(256), 0, st, (uint8_t *)dst, n, seed, first);
    return hipGetLastError();
}

hipError_t launch_gen_normal(float *dst, uint64_t n, uint64_t seed, uint64_t first, float mean,
                             float stdv, hipStream_t st) {
    if (n == 0) return hipSuccess;
    dim3 grid((unsigned)((n + 255) / 256));
    hipLaunchKernelGGL(k_gen_normal, grid, dim3(256), 0, st, dst, n, seed, first, mean, stdv);
    return hipGetLastError();
}

hipError_t launch_gen_logits(float *dst, int M, int E, uint64_t seed, int kind, double param,
                             double hot_value, hipStream_t st) {
    uint64_t n = (uint64_t)M * (uint64_t)E;
    if (n == 0) return hipSuccess;
    dim3 grid((unsigned)((n + 255) / 256));
    hipLaunchKernelGGL(k_gen_logits, grid, dim3(256), 0, st, dst, M, E, seed, kind, param, hot_value);
    return hipGetLastError();
}

} // namespace moe
