/*
 * moe_oracle.c -- CPU oracle for the MoE expert-FFN hot path (TEST INFRASTRUCTURE ONLY).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this file's
 * library, and only as the checker or as the reported CPU baseline.  The product library
 * (moe-680m_amd/) never links or calls it.
 *
 * Each function names the reference lines it restates.  The reference's literal shaders
 * cannot serve as numeric oracles (their tiled kernels index with gl_GlobalInvocationID
 * where gl_WorkGroupID is meant, their _m1 kernels store f16 through racy 32-bit
 * read-modify-writes, and f16 activations overflow under the seeded distribution), so the
 * oracle restates the intended algorithm in f64, as listed in moe_oracle.h.
 *
 * Compiled with -ffp-contract=off: the seeded generator below must produce the same bits
 * as the device generator, so no multiply-add may be fused behind the source's back.
 */
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ggml kvalues_iq4nl: the 16-entry non-linear codebook of IQ4_NL / IQ4_XS. */
static const int8_t KVALUES[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                   1,    13,   25,  38,  53,  69,  89,  113};

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------ f16 / bf16 */

/* Exact IEEE binary16 decode.  The reference's GLSL decoder flushes subnormals
 * (shaders/common.glsl:20-35); this build decodes them exactly, as gfx950's
 * v_cvt_f32_f16 does. */
float orc_f16_to_f32(uint16_t h) {
    uint32_t s = (uint32_t)(h >> 15) & 1u, e = (uint32_t)(h >> 10) & 31u, m = (uint32_t)h & 1023u;
    float v;
    if (e == 0)
        v = ldexpf((float)m, -24);
    else if (e == 31)
        v = m ? NAN : INFINITY;
    else
        v = ldexpf((float)(m | 1024u), (int)e - 25);
    return s ? -v : v;
}

/* f32 -> f16 with round-to-nearest-even, subnormals and overflow to inf. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ex = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (ex == 0xFF) return (uint16_t)(sign | 0x7C00u | (man ? 0x200u : 0u));
    int e = (int)ex - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m = man | 0x800000u;
        int shift = 14 - e; /* 14..24 */
        uint32_t q = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++; /* may carry into inf: correct */
    return (uint16_t)(sign | q);
}

uint16_t orc_f32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
    uint32_t lsb = (x >> 16) & 1u;
    x += 0x7FFFu + lsb;
    return (uint16_t)(x >> 16);
}

float orc_bf16_to_f32(uint16_t b) {
    uint32_t x = (uint32_t)b << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* ------------------------------------------------------------------ IQ4_XS */

/* ggml block_iq4_xs: f16 d @0 | u16 scales_h @2 | u8 scales_l[4] @4 | u8 qs[128] @8.
 * Sub-block ib (32 weights): ls = scales_l nibble ib | 2 bits of scales_h << 4,
 * value = d*(ls-32) * kvalues[nibble]; byte j of the sub-block holds weight j (low nibble)
 * and weight j+16 (high nibble).  This replaces the reference's 36-byte block decoder
 * (shaders/common.glsl:61-86, src/inference.rs:196-210). */
void orc_dequant_iq4xs(const uint8_t *blocks, size_t n_sb, float *out) {
    for (size_t b = 0; b < n_sb; ++b) {
        const uint8_t *p = blocks + ORC_SB_BYTES * b;
        float d = orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
        unsigned sh = (unsigned)(p[2] | (p[3] << 8));
        for (int ib = 0; ib < 8; ++ib) {
            int ls = ((p[4 + ib / 2] >> (4 * (ib % 2))) & 0xF) | (int)(((sh >> (2 * ib)) & 3u) << 4);
            float dl = d * (float)(ls - 32);
            for (int j = 0; j < 16; ++j) {
                uint8_t q = p[8 + 16 * ib + j];
                out[ORC_QK * b + 32 * ib + j] = dl * (float)KVALUES[q & 0xF];
                out[ORC_QK * b + 32 * ib + 16 + j] = dl * (float)KVALUES[q >> 4];
            }
        }
    }
}

/* ------------------------------------------------------------------ router */

static inline double sel_key(float v) {
    if (v != v) return -INFINITY; /* NaN never wins */
    return (double)v;             /* -0 == +0 under double compare */
}

/* Softmax + top-8, restating shaders/router_topk.comp:31-92 (max, exp(l-max), sum,
 * normalise; insertion with strict '>' so the lower index wins ties; descending order)
 * and src/router.rs:23-51 (same softmax; 8 selected with their probabilities).
 * Selection is done on logits, which softmax orders identically.  Shared expert: the
 * reference puts it at entry 0 with id 0 (router_topk.comp:64, router.rs:50), colliding
 * with routed expert 0; here it is slot 8 with id E, its own bucket. */
void orc_router_topk(const float *logits, int M, int E, int mode, uint16_t *ids, float *w) {
    for (int t = 0; t < M; ++t) {
        const float *l = logits + (size_t)t * E;
        int sel[ORC_TOPK];
        for (int r = 0; r < ORC_TOPK; ++r) {
            int best = -1;
            double bk = 0;
            for (int i = 0; i < E; ++i) {
                int used = 0;
                for (int q = 0; q < r; ++q) used |= (sel[q] == i);
                if (used) continue;
                double k = sel_key(l[i]);
                if (best < 0 || k > bk) { best = i; bk = k; }
            }
            sel[r] = best;
        }
        double mx = sel_key(l[sel[0]]);
        double Z = 0;
        for (int i = 0; i < E; ++i) {
            double k = sel_key(l[i]);
            Z += (k == mx) ? 1.0 : exp(k - mx);
        }
        double S8 = 0;
        double e8[ORC_TOPK];
        for (int r = 0; r < ORC_TOPK; ++r) {
            double k = sel_key(l[sel[r]]);
            e8[r] = (k == mx) ? 1.0 : exp(k - mx);
            S8 += e8[r];
        }
        for (int r = 0; r < ORC_TOPK; ++r) {
            ids[(size_t)t * ORC_SLOTS + r] = (uint16_t)sel[r];
            double p = (mode == ORC_W_RENORM) ? e8[r] / S8 : e8[r] / Z;
            w[(size_t)t * ORC_SLOTS + r] = (float)p;
        }
        ids[(size_t)t * ORC_SLOTS + 8] = (uint16_t)E;
        w[(size_t)t * ORC_SLOTS + 8] = 1.0f;
    }
}

/* ------------------------------------------------------------------ bucket fill */

/* Counting sort restating src/router.rs:55-97: count per bucket, exclusive prefix sum,
 * then a stable fill visiting tokens in order and, inside a token, routed slots 0..7
 * then the shared slot.  Buckets: 0..E-1 routed, E shared (the reference folds the
 * shared expert into bucket 0, router.rs:67). */
void orc_bucket_fill(const uint16_t *ids, const float *w, int M, int E, uint32_t *ranges,
                     uint16_t *sorted_tok, float *sorted_w, uint32_t *pos) {
    int nb = E + 1;
    uint32_t *cursor = (uint32_t *)calloc((size_t)nb + 1, sizeof(uint32_t));
    for (int i = 0; i <= nb; ++i) ranges[i] = 0;
    for (int t = 0; t < M; ++t)
        for (int s = 0; s < ORC_SLOTS; ++s) ranges[ids[(size_t)t * ORC_SLOTS + s] + 1]++;
    for (int e = 0; e < nb; ++e) ranges[e + 1] += ranges[e];
    for (int e = 0; e <= nb; ++e) cursor[e] = ranges[e];
    for (int t = 0; t < M; ++t)
        for (int s = 0; s < ORC_SLOTS; ++s) {
            int e = ids[(size_t)t * ORC_SLOTS + s];
            uint32_t p = cursor[e]++;
            sorted_tok[p] = (uint16_t)t;
            sorted_w[p] = w[(size_t)t * ORC_SLOTS + s];
            if (pos) pos[(size_t)t * ORC_SLOTS + s] = p;
        }
    free(cursor);
}

/* ------------------------------------------------------------------ FFN */

static double dot_f32_f64(const float *a, const double *b, int n) {
    double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 8 <= n; i += 8)
        for (int j = 0; j < 8; ++j) acc[j] += (double)a[i + j] * b[i + j];
    for (; i < n; ++i) acc[0] += (double)a[i] * b[i];
    return ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
}

static inline double silu(double v) { return v / (1.0 + exp(-v)); }

/* RMSNorm with unit gain and eps 1e-6, restating shaders/rms_norm.comp:30-46. */
void orc_rmsnorm(const float *x, int H, double *out) {
    double ss = 0;
    for (int k = 0; k < H; ++k) ss += (double)x[k] * x[k];
    double inv = 1.0 / sqrt(ss / H + 1e-6);
    for (int k = 0; k < H; ++k) out[k] = x[k] * inv;
}

/* Router gate GEMV, restating shaders/router.comp:21-61 (logits = x . Wg, dispatched at
 * src/inference.rs:598-605) with Wg rows = experts (the [out][in] convention of the expert
 * matrices): logits[t][e] = sum_k xin[t][k] * Wg[e][k], xin = x or RMSNorm(x).  f64 sums of
 * the f32 weights W [E][H]; the output is the f64 value rounded to f32. */
void orc_router_gemv_f32(const float *W, int H, int E, const float *x, int M, int flags, float *logits) {
#pragma omp parallel
    {
        double *xin = (double *)malloc((size_t)H * sizeof(double));
#pragma omp for schedule(static)
        for (int t = 0; t < M; ++t) {
            if (flags & ORC_FFN_RMSNORM)
                orc_rmsnorm(x + (size_t)t * H, H, xin);
            else
                for (int k = 0; k < H; ++k) xin[k] = x[(size_t)t * H + k];
            for (int e = 0; e < E; ++e) logits[(size_t)t * E + e] = (float)dot_f32_f64(W + (size_t)e * H, xin, H);
        }
        free(xin);
    }
}

/* The same on an IQ4_XS gate matrix (wg: E*H/256 super-blocks), decoded exactly first. */
void orc_router_gemv(const uint8_t *wg, int H, int E, const float *x, int M, int flags, float *logits) {
    size_t nw = (size_t)E * H;
    float *W = (float *)malloc(nw * 4);
    orc_dequant_iq4xs(wg, nw / ORC_QK, W);
    orc_router_gemv_f32(W, H, E, x, M, flags, logits);
    free(W);
}

/* gate||up then SiLU*up then down, restating w1_w3_fused_m1.comp:30-52 (gate from W1,
 * up from W3), w2_scatter.comp:31-42 (A = silu(gate)*up) and :44-57 (down product). */
static void expert_rows(const float *W1, const float *W3, const float *W2, int H, int I,
                        const double *xin, double *h, double *y) {
    for (int n = 0; n < I; ++n) {
        double g = dot_f32_f64(W1 + (size_t)n * H, xin, H);
        double u = dot_f32_f64(W3 + (size_t)n * H, xin, H);
        h[n] = silu(g) * u;
    }
    for (int n = 0; n < H; ++n) y[n] = dot_f32_f64(W2 + (size_t)n * I, h, I);
}

void orc_expert_forward(const uint8_t *w1, const uint8_t *w3, const uint8_t *w2, int H, int I,
                        const float *x, double *y) {
    size_t nw = (size_t)H * I;
    float *W1 = (float *)malloc(nw * 4), *W3 = (float *)malloc(nw * 4), *W2 = (float *)malloc(nw * 4);
    double *xin = (double *)malloc((size_t)H * 8), *h = (double *)malloc((size_t)I * 8);
    orc_dequant_iq4xs(w1, nw / ORC_QK, W1);
    orc_dequant_iq4xs(w3, nw / ORC_QK, W3);
    orc_dequant_iq4xs(w2, nw / ORC_QK, W2);
    for (int k = 0; k < H; ++k) xin[k] = x[k];
    expert_rows(W1, W3, W2, H, I, xin, h, y);
    free(W1); free(W3); free(W2); free(xin); free(h);
}

static const uint8_t *expert_ptr(const uint8_t *base, size_t stride, const uint8_t *shared, int e,
                                 int E) {
    return e == E ? shared : base + (size_t)e * stride;
}

/* Whole layer.  Combine restates src/inference.rs:736-762: every selected expert's output
 * is scaled by its weight times the dispatch scale (1/9 there, c here) and summed onto
 * the hidden state; the shared expert enters with weight 1.  Experts are evaluated once
 * each for all tokens that chose them, then summed per token in slot order. */
/* Slot s of a token repeats an id of one of its earlier slots (such a slot is dropped). */
static int repeats_earlier_slot(const uint16_t *tok_ids, int s) {
    for (int s2 = 0; s2 < s; ++s2)
        if (tok_ids[s2] == tok_ids[s]) return 1;
    return 0;
}

void orc_moe_ffn(const orc_layer *L, int H, int I, int E, const float *x, const uint16_t *ids,
                 const float *w, int M, double c, int flags, float *y) {
    int nb = E + 1;
    double *xin = (double *)malloc((size_t)M * H * sizeof(double));
    double *ys = (double *)calloc((size_t)M * ORC_SLOTS * H, sizeof(double));
    for (int t = 0; t < M; ++t) {
        if (flags & ORC_FFN_RMSNORM)
            orc_rmsnorm(x + (size_t)t * H, H, xin + (size_t)t * H);
        else
            for (int k = 0; k < H; ++k) xin[(size_t)t * H + k] = x[(size_t)t * H + k];
    }
    /* unique experts used */
    int *used = (int *)calloc((size_t)nb, sizeof(int));
    int *list = (int *)malloc((size_t)nb * sizeof(int));
    int nl = 0;
    for (int t = 0; t < M; ++t)
        for (int s = 0; s < ORC_SLOTS; ++s) {
            int e = ids[(size_t)t * ORC_SLOTS + s];
            if (e >= 0 && e < nb && !used[e]) { used[e] = 1; list[nl++] = e; }
        }
    size_t nw = (size_t)H * I;
#pragma omp parallel
    {
        float *W1 = (float *)malloc(nw * 4), *W3 = (float *)malloc(nw * 4), *W2 = (float *)malloc(nw * 4);
        double *h = (double *)malloc((size_t)I * 8);
#pragma omp for schedule(dynamic, 1)
        for (int li = 0; li < nl; ++li) {
            int e = list[li];
            orc_dequant_iq4xs(expert_ptr(L->w1, L->w1_stride, L->shared_w1, e, E), nw / ORC_QK, W1);
            orc_dequant_iq4xs(expert_ptr(L->w3, L->w3_stride, L->shared_w3, e, E), nw / ORC_QK, W3);
            orc_dequant_iq4xs(expert_ptr(L->w2, L->w2_stride, L->shared_w2, e, E), nw / ORC_QK, W2);
            for (int t = 0; t < M; ++t)
                for (int s = 0; s < ORC_SLOTS; ++s)
                    if (ids[(size_t)t * ORC_SLOTS + s] == e && !repeats_earlier_slot(ids + (size_t)t * ORC_SLOTS, s))
                        expert_rows(W1, W3, W2, H, I, xin + (size_t)t * H, h,
                                    ys + ((size_t)t * ORC_SLOTS + s) * H);
        }
        free(W1); free(W3); free(W2); free(h);
    }
    for (int t = 0; t < M; ++t)
        for (int n = 0; n < H; ++n) {
            double acc = 0;
            for (int s = 0; s < ORC_SLOTS; ++s)
                acc += (double)w[(size_t)t * ORC_SLOTS + s] * ys[((size_t)t * ORC_SLOTS + s) * H + n];
            double base = (flags & ORC_FFN_ACCUMULATE) ? (double)y[(size_t)t * H + n] : 0.0;
            y[(size_t)t * H + n] = (float)(base + c * acc);
        }
    free(xin); free(ys); free(used); free(list);
}

/* The same layer in f32 (f32 products and sums) with OpenMP over the output rows of each
 * expert, rows decoded as they are used: the CPU baseline's timed path.  Checked against
 * orc_moe_ffn (f64) by the CPU tests; not a checker itself. */
static void dequant_row(const uint8_t *row, int n_sb, float *out) { orc_dequant_iq4xs(row, (size_t)n_sb, out); }

void orc_moe_ffn_f32(const orc_layer *L, int H, int I, int E, const float *x, const uint16_t *ids,
                     const float *w, int M, float c, int flags, float *y) {
    const int nb = E + 1;
    const size_t rb1 = (size_t)H / ORC_QK * ORC_SB_BYTES, rb2 = (size_t)I / ORC_QK * ORC_SB_BYTES;
    float *xin = (float *)malloc((size_t)M * H * sizeof(float));
    float *out = (float *)calloc((size_t)M * H, sizeof(float));
    float *h = (float *)malloc((size_t)M * I * sizeof(float));
    int *tok = (int *)malloc((size_t)M * sizeof(int));
    float *tw = (float *)malloc((size_t)M * sizeof(float));
    for (int t = 0; t < M; ++t) {
        const float *xt = x + (size_t)t * H;
        float inv = 1.0f;
        if (flags & ORC_FFN_RMSNORM) {
            float ss = 0.f;
            for (int k = 0; k < H; ++k) ss += xt[k] * xt[k];
            inv = 1.0f / sqrtf(ss / (float)H + 1e-6f);
        }
        for (int k = 0; k < H; ++k) xin[(size_t)t * H + k] = xt[k] * inv;
    }
    for (int e = 0; e < nb; ++e) {
        int nt = 0;
        for (int t = 0; t < M; ++t)
            for (int s = 0; s < ORC_SLOTS; ++s)
                if (ids[(size_t)t * ORC_SLOTS + s] == e && !repeats_earlier_slot(ids + (size_t)t * ORC_SLOTS, s)) {
                    tok[nt] = t;
                    tw[nt++] = w[(size_t)t * ORC_SLOTS + s];
                }
        if (!nt) continue;
        const uint8_t *W1 = expert_ptr(L->w1, L->w1_stride, L->shared_w1, e, E);
        const uint8_t *W3 = expert_ptr(L->w3, L->w3_stride, L->shared_w3, e, E);
        const uint8_t *W2 = expert_ptr(L->w2, L->w2_stride, L->shared_w2, e, E);
#pragma omp parallel
        {
            float *r1 = (float *)malloc((size_t)H * 4), *r3 = (float *)malloc((size_t)H * 4);
#pragma omp for schedule(static)
            for (int n = 0; n < I; ++n) {
                dequant_row(W1 + (size_t)n * rb1, H / ORC_QK, r1);
                dequant_row(W3 + (size_t)n * rb1, H / ORC_QK, r3);
                for (int j = 0; j < nt; ++j) {
                    const float *xt = xin + (size_t)tok[j] * H;
                    float g = 0.f, u = 0.f;
                    for (int k = 0; k < H; ++k) {
                        g += r1[k] * xt[k];
                        u += r3[k] * xt[k];
                    }
                    h[(size_t)j * I + n] = g / (1.0f + expf(-g)) * u;
                }
            }
#pragma omp for schedule(static)
            for (int n = 0; n < H; ++n) {
                dequant_row(W2 + (size_t)n * rb2, I / ORC_QK, r1);
                for (int j = 0; j < nt; ++j) {
                    float a = 0.f;
                    for (int k = 0; k < I; ++k) a += r1[k] * h[(size_t)j * I + k];
                    out[(size_t)tok[j] * H + n] += c * tw[j] * a;
                }
            }
            free(r1); free(r3);
        }
    }
    for (size_t i = 0; i < (size_t)M * H; ++i) y[i] = ((flags & ORC_FFN_ACCUMULATE) ? y[i] : 0.f) + out[i];
    free(xin); free(out); free(h); free(tok); free(tw);
}

/* ------------------------------------------------------------------ generator */
/* Counter-based, so any slice of any stream can be produced independently.  The device
 * generator (moe-680m_amd/csrc) implements the same specification separately; tests
 * compare the two.  Only IEEE basic operations (+ - * / sqrt, frexp, floor) are used, with
 * no contraction, so both sides produce the same bits. */

uint64_t orc_mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t orc_rng(uint64_t seed, uint64_t i) { return orc_mix64(seed ^ orc_mix64(i)); }

/* natural log for x > 0: x = m 2^e with m in [sqrt(1/2), sqrt(2)), log m = 2 atanh(s). */
double orc_glog(double x) {
    int e;
    double m = frexp(x, &e);
    if (m < 0.70710678118654752440) { m = m * 2.0; e -= 1; }
    double s = (m - 1.0) / (m + 1.0);
    double s2 = s * s;
    double p = 1.0 / 23.0;
    for (int k = 21; k >= 1; k -= 2) { p = p * s2; p = p + 1.0 / (double)k; }
    double lm = 2.0 * s * p;
    return (double)e * 0.69314718055994530942 + lm;
}

static double taylor_sin(double a) {
    double a2 = a * a, term = a, sum = a;
    for (int k = 1; k <= 11; ++k) { term = -term * a2 / (double)((2 * k) * (2 * k + 1)); sum = sum + term; }
    return sum;
}
static double taylor_cos(double a) {
    double a2 = a * a, term = 1.0, sum = 1.0;
    for (int k = 1; k <= 11; ++k) { term = -term * a2 / (double)((2 * k - 1) * (2 * k)); sum = sum + term; }
    return sum;
}

/* cos(2 pi u) */
double orc_gcos2pi(double u) {
    double wv = u - floor(u + 0.5);
    wv = fabs(wv);
    double sgn = 1.0;
    if (wv > 0.25) { wv = 0.5 - wv; sgn = -1.0; }
    const double TWO_PI = 6.283185307179586476925;
    double r;
    if (wv > 0.125) r = taylor_sin(TWO_PI * (0.25 - wv));
    else r = taylor_cos(TWO_PI * wv);
    return sgn * r;
}

static inline double u01_open(uint64_t r) { return (double)((r >> 11) + 1) * 0x1.0p-53; }
static inline double u01(uint64_t r) { return (double)(r >> 11) * 0x1.0p-53; }

static double box_muller(uint64_t r1, uint64_t r2) {
    double u1 = u01_open(r1), u2 = u01(r2);
    return sqrt(-2.0 * orc_glog(u1)) * orc_gcos2pi(u2);
}

double orc_normal(uint64_t seed, uint64_t i) {
    return box_muller(orc_rng(seed, 2 * i), orc_rng(seed, 2 * i + 1));
}

/* Super-block b uses words rng(seed, 32b + j): j 0..15 -> the 128 nibble bytes (little
 * endian), j 16 -> eight 6-bit scales, j 17,18 -> d = f16(f32(|N(0,1)| * 2e-3)). */
void orc_gen_iq4xs(uint64_t seed, uint64_t first, size_t n, uint8_t *out) {
#pragma omp parallel for schedule(static)
    for (long long bi = 0; bi < (long long)n; ++bi) {
        uint64_t b = first + (uint64_t)bi;
        uint8_t *p = out + ORC_SB_BYTES * (size_t)bi;
        for (int j = 0; j < 16; ++j) {
            uint64_t r = orc_rng(seed, 32 * b + (uint64_t)j);
            for (int k = 0; k < 8; ++k) p[8 + 8 * j + k] = (uint8_t)(r >> (8 * k));
        }
        uint64_t rs = orc_rng(seed, 32 * b + 16);
        unsigned sh = 0;
        uint8_t sl[4] = {0, 0, 0, 0};
        for (int ib = 0; ib < 8; ++ib) {
            unsigned ls = (unsigned)(rs >> (6 * ib)) & 63u;
            sl[ib / 2] |= (uint8_t)((ls & 15u) << (4 * (ib % 2)));
            sh |= (ls >> 4) << (2 * ib);
        }
        double z = box_muller(orc_rng(seed, 32 * b + 17), orc_rng(seed, 32 * b + 18));
        double dv = fabs(z) * 2e-3;
        uint16_t dh = orc_f32_to_f16((float)dv);
        p[0] = (uint8_t)(dh & 0xFF);
        p[1] = (uint8_t)(dh >> 8);
        p[2] = (uint8_t)(sh & 0xFF);
        p[3] = (uint8_t)(sh >> 8);
        for (int k = 0; k < 4; ++k) p[4 + k] = sl[k];
    }
}

void orc_gen_normal(uint64_t seed, uint64_t first, size_t n, float mean, float std, float *out) {
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; ++i) {
        double z = orc_normal(seed, first + (uint64_t)i);
        double v = z * (double)std;
        v = v + (double)mean;
        out[i] = (float)v;
    }
}

#define TAG_PERM 0x5045524Dull
#define TAG_HOTE 0x484F5445ull
#define TAG_HOTT 0x484F5454ull

int orc_zipf_rank(uint64_t seed, int E, int e) {
    uint64_t ke = orc_rng(seed ^ TAG_PERM, (uint64_t)e);
    int rank = 1;
    for (int j = 0; j < E; ++j) {
        uint64_t kj = orc_rng(seed ^ TAG_PERM, (uint64_t)j);
        if (kj < ke || (kj == ke && j < e)) rank++;
    }
    return rank;
}

int orc_hot_expert(uint64_t seed, int E) { return (int)(orc_rng(seed ^ TAG_HOTE, 0) % (uint64_t)E); }

void orc_gen_logits(uint64_t seed, int M, int E, int kind, double param, double hot_value,
                    float *out) {
    double *bias = (double *)calloc((size_t)E, sizeof(double));
    if (kind == 1)
        for (int e = 0; e < E; ++e) {
            double lr = orc_glog((double)orc_zipf_rank(seed, E, e));
            bias[e] = -param * lr;
        }
    int hot = orc_hot_expert(seed, E);
    for (int t = 0; t < M; ++t) {
        int is_hot = (kind == 2) && (u01(orc_rng(seed ^ TAG_HOTT, (uint64_t)t)) < param);
        for (int e = 0; e < E; ++e) {
            double z = orc_normal(seed, (uint64_t)t * E + (uint64_t)e);
            double v = z + bias[e];
            if (is_hot && e == hot) v = hot_value;
            out[(size_t)t * E + e] = (float)v;
        }
    }
    free(bias);
}
