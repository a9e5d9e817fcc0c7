/*
 * moe_oracle.h -- CPU oracle for the MoE expert-FFN hot path of herlangga72/moe-680m.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links, loads or calls
 * this code.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
 * it, and only as the checker (or as the timed CPU baseline), never as a product path.
 *
 * What it restates (citations are path:line in the reference tree):
 *   - router gate GEMV            shaders/router.comp:21-61, src/inference.rs:598-605
 *   - router softmax + top-8      shaders/router_topk.comp:31-92, src/router.rs:23-51
 *   - prefix-sum bucket fill      src/router.rs:55-97
 *   - gate||up GEMV, fused SiLU   shaders/w1_w3_fused_m1.comp:30-52, shaders/w1_w3_fused.comp:47-48,
 *                                 shaders/w2_scatter.comp:31-42, shaders/common.glsl:106-108
 *   - down-proj + weighted scatter shaders/w2_scatter.comp:67-86, shaders/w2_scatter_m1.comp:53-62
 *   - combine (shared first, x1/9) src/inference.rs:736-762, src/inference.rs:720,750
 *   - RMSNorm (eps 1e-6, no gain)  shaders/rms_norm.comp:30-46
 * The weight codec is GGML IQ4_XS (136-byte super-blocks of 256 weights), which the
 * reference names but does not implement (its shaders decode a 36-byte/32-weight block,
 * shaders/common.glsl:61-86).  The codec follows ggml's published block_iq4_xs /
 * dequantize_row_iq4_xs definition; no copy of ggml is present here, so the codec is
 * pinned by closed-form known-answer tests rather than by reference vectors.
 *
 * Arithmetic: dequantised weights are exact f32 (products of <=23 significant bits);
 * every dot product, softmax and norm is accumulated in f64.
 */
#ifndef MOE_ORACLE_H
#define MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QK 256          /* weights per IQ4_XS super-block */
#define ORC_SB_BYTES 136    /* bytes per IQ4_XS super-block   */
#define ORC_TOPK 8
#define ORC_SLOTS 9         /* 8 routed + 1 shared */

enum { ORC_W_REF = 0, ORC_W_RENORM = 1 };
enum { ORC_FFN_ACCUMULATE = 1, ORC_FFN_RMSNORM = 2 };

/* IEEE binary16 <-> binary32, exact decode including subnormals, RNE encode. */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
/* f32 -> bf16 bits, round to nearest even (NaN kept quiet). */
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t b);

/* GGML IQ4_XS decode of n_sb super-blocks into out[256*n_sb]. */
void orc_dequant_iq4xs(const uint8_t *blocks, size_t n_sb, float *out);

/* Router: logits f32 [M][E] -> ids u16 [M][9], w f32 [M][9].
 * Slots 0..7: the 8 largest logits ordered by (logit desc, index asc); NaN counts as -inf
 * and -0 as +0.  Slot 8: the shared expert, id E, weight 1.
 * mode ORC_W_REF: w = softmax probability; ORC_W_RENORM: w renormalised over the 8. */
void orc_router_topk(const float *logits, int M, int E, int mode, uint16_t *ids, float *w);

/* Bucket fill over E+1 buckets (bucket E = shared expert).
 * ranges[E+2] exclusive prefix sum of counts; sorted_tok / sorted_w [9M] in bucket order,
 * ascending token inside a bucket; pos[M][9] (may be NULL) = sorted index of slot (t,s). */
void orc_bucket_fill(const uint16_t *ids, const float *w, int M, int E,
                     uint32_t *ranges, uint16_t *sorted_tok, float *sorted_w, uint32_t *pos);

/* One layer's expert table.  Routed expert e: W1 at w1 + e*w1_stride, etc.
 * Shared expert (id E): shared_w1/w3/w2.  Row-major [out][in] IQ4_XS, rows are outputs. */
typedef struct {
    const uint8_t *w1, *w3, *w2;
    size_t w1_stride, w3_stride, w2_stride;
    const uint8_t *shared_w1, *shared_w3, *shared_w2;
} orc_layer;

/* Full MoE FFN of one layer for M tokens (Appendix-A semantics):
 *   xin = flags&RMSNORM ? x / sqrt(mean(x^2) + 1e-6) : x
 *   y_e = W2_e (silu(W1_e xin) * (W3_e xin))
 *   out = c * sum_{s<9} w[s] * y_{ids[s]}
 *   y   = flags&ACCUMULATE ? y + out : out
 * A slot whose id is above E, or repeats an id of an earlier slot of the same token, adds
 * nothing (the rule the product's bucket fill and decode kernels apply; the reference's
 * router never produces either).  x and y may alias.  Accumulation in f64. */
void orc_moe_ffn(const orc_layer *L, int H, int I, int E, const float *x, const uint16_t *ids,
                 const float *w, int M, double c, int flags, float *y);

/* orc_moe_ffn in f32 arithmetic with OpenMP over each expert's output rows: the timed CPU
 * baseline (a port of the same algorithm), checked against orc_moe_ffn; not a checker. */
void orc_moe_ffn_f32(const orc_layer *L, int H, int I, int E, const float *x, const uint16_t *ids,
                     const float *w, int M, float c, int flags, float *y);

/* Router gate GEMV: logits[t][e] = sum_k xin[t][k] * Wg[e][k] (f64 sum, rounded to f32),
 * xin = flags & ORC_FFN_RMSNORM ? RMSNorm(x_t) : x_t.  wg: IQ4_XS [E][H], rows = experts. */
void orc_router_gemv(const uint8_t *wg, int H, int E, const float *x, int M, int flags, float *logits);
void orc_router_gemv_f32(const float *W, int H, int E, const float *x, int M, int flags, float *logits);

/* Single expert on one row, f64 out (for fine-grained tests). */
void orc_expert_forward(const uint8_t *w1, const uint8_t *w3, const uint8_t *w2, int H, int I,
                        const float *x, double *y);

/* ---- seeded generator (independent restatement of the device generator's spec) ---- */
uint64_t orc_mix64(uint64_t z);
uint64_t orc_rng(uint64_t seed, uint64_t i);
double orc_normal(uint64_t seed, uint64_t i);
double orc_glog(double x);
double orc_gcos2pi(double u);
/* Super-blocks first..first+n-1 of the stream 'seed' -> out[136*n]. */
void orc_gen_iq4xs(uint64_t seed, uint64_t first, size_t n, uint8_t *out);
/* out[i] = (float)(mean + std * normal(seed, first + i)). */
void orc_gen_normal(uint64_t seed, uint64_t first, size_t n, float mean, float std, float *out);
/* Router logits [M][E]: N(0,1) from stream seed (element index t*E+e) plus a bias:
 *   kind 0: none
 *   kind 1: Zipf(s)  bias_e = -s * log(rank_e), rank from a seeded permutation (seed^PERM)
 *   kind 2: hot      with probability p (seeded per token), logit[hot] = hot_value  */
void orc_gen_logits(uint64_t seed, int M, int E, int kind, double param, double hot_value,
                    float *out);
int orc_zipf_rank(uint64_t seed, int E, int e);
int orc_hot_expert(uint64_t seed, int E);

/* Convenience: RMSNorm of one row into f64 buffer. */
void orc_rmsnorm(const float *x, int H, double *out);

int orc_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
