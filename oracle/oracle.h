/*
 * oracle.h -- CPU restatement of the ggml CPU-backend arithmetic that the
 * diffusers-cpp Flux2 modules emit for the DiT elementwise/reduction chain.
 *
 * This is the ORACLE: test infrastructure only.  Only the tests, the smoke
 * check and the CPU-baseline leg of the benchmark may load it, and only as
 * the thing results are checked against (or, for the baseline, timed).  The
 * product library never links or calls it.
 *
 * ggml itself (https://github.com/ggml-org/ggml, the reference's un-vendored
 * submodule `ggml/`, pinned commit unknown) is not available, so each
 * function restates ggml's published CPU algorithm and names the reference
 * call site it stands in for.  Rounding follows the literal C expression
 * order (the library is compiled with -ffp-contract=off).
 *
 * Conventions: rows are contiguous, `cols` elements each, unless a stride is
 * given.  Positions are int32.  bf16/fp16 values travel as uint16_t bit
 * patterns.  `nthreads` <= 0 means "use the OpenMP default".
 */
#ifndef DIT_ORACLE_H
#define DIT_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- seeded generator: std::mt19937_64 + in-repo Box-Muller ------------ */
uint64_t or_mt64_nth(uint64_t seed, uint64_t n);           /* n-th output, 1-based */
void or_randn_f32(uint64_t seed, int64_t n, float mean, float std, float *out);
void or_rand_int32(uint64_t seed, int64_t n, int32_t lo, int32_t hi, int32_t *out);
/* Hash-drawn test weights (integer arithmetic only): Q8_0 blocks of a
 * [rows, cols] Linear weight and RMSNorm weights, keyed by seed and the
 * parameter path (the rule is stated in oracle.c). */
uint64_t or_splitmix64(uint64_t z);
uint64_t or_fnv1a64(const char *s);
uint64_t or_hash_key(uint64_t seed, const char *path);
void or_hash_q8_0(uint64_t seed, const char *path, int64_t rows, int64_t cols, uint8_t *dst, int nthreads);
void or_hash_norm_weight(uint64_t seed, const char *path, int64_t n, float *out);

/* ---- number formats ----------------------------------------------------- */
float    or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);                            /* RNE */
float    or_bf16_to_f32(uint16_t h);
uint16_t or_f32_to_bf16(float f);                           /* RNE, NaN quieted */
void or_f32_to_bf16_n(const float *x, int64_t n, uint16_t *y);
void or_bf16_to_f32_n(const uint16_t *x, int64_t n, float *y);
void or_round_bf16_n(const float *x, int64_t n, float *y);  /* x -> bf16 -> f32 */

/* ---- single ggml ops (fp32) -------------------------------------------- */
void or_norm_f32(const float *x, int64_t rows, int64_t cols, float eps, float *y, int nthreads);
void or_rms_norm_f32(const float *x, int64_t rows, int64_t cols, float eps, float *y, int nthreads);
void or_sigmoid_f32(const float *x, int64_t n, float *y);
void or_scale_f32(const float *x, int64_t n, float s, float *y);

/* ggml binary op with src1 broadcast into src0 (dst has src0's shape).
 * op: 0 add, 1 sub, 2 mul, 3 div.  ne/nb are ggml-order (ne[0] fastest),
 * nb in bytes; dst is written contiguous. */
void or_binary_f32(int op,
                   const float *a, const int64_t ne_a[4], const int64_t nb_a[4],
                   const float *b, const int64_t ne_b[4], const int64_t nb_b[4],
                   float *dst);

/* ggml_concat along ggml dim `dim` of two contiguous tensors. */
void or_concat_f32(const float *a, const int64_t ne_a[4],
                   const float *b, const int64_t ne_b[4], int dim, float *dst);

/* RoPE cache for one position (ggml_rope_cache_init with ext_factor = 0):
 * cache[2i] = cos(theta_i), cache[2i+1] = sin(theta_i) for i < ne0/2, with
 * theta_0 = p * freq_scale and theta_{i+1} = theta_i * powf(base, -2/n_dims). */
void or_rope_cache(float p, int n_dims, int64_t ne0, float freq_base,
                   float freq_scale, float attn_factor, float *cache);

/* ggml_rope_ext, mode NORMAL, ext_factor 0, no freq factors, on a strided
 * 4-D src (ne/nb ggml order, nb in bytes); pos has ne[2] entries; dst is
 * contiguous [ne3][ne2][ne1][ne0]. Dims >= n_dims are copied through. */
void or_rope_normal_f32(const float *x, const int64_t ne[4], const int64_t nb[4],
                        const int32_t *pos, int n_dims, float freq_base,
                        float freq_scale, float attn_factor, float *dst);

/* ---- chains, composed exactly as the reference's modules emit them ----- */

/* LayerNorm(no affine) then `(1+scale)*n + shift`:
 * y = add(mul(norm(x), add(scale, 1.0f)), shift). */
void or_adaln_f32(const float *x, int64_t rows, int64_t cols,
                  const float *shift, const float *scale, float eps, float *y,
                  int nthreads);

/* RMSNorm(q) * w, then the 4-section Flux2PosEmbed rotation.
 * x, y: [tokens][heads][n_axes*axis_dim]; w: [head_dim];
 * pos: [tokens][pos_stride] int32, axis a uses column a. */
void or_qk_rmsnorm_rope_f32(const float *x, int64_t tokens, int64_t heads,
                            int64_t head_dim, const float *w, float eps,
                            const int32_t *pos, int64_t pos_stride, int n_axes,
                            int axis_dim, float freq_base, float *y, int nthreads);

/* Flux2SwiGLU: y = mul(mul(g, sigmoid(g)), u); row strides in elements. */
void or_swiglu_f32(const float *g, int64_t g_stride, const float *u, int64_t u_stride,
                   int64_t rows, int64_t cols, float *y, int nthreads);

/* gated residual y = add(h, mul(o, gate)), gate broadcast over rows. */
void or_gated_residual_f32(const float *h, const float *o, const float *gate,
                           int64_t rows, int64_t cols, float *y, int nthreads);

/* GroupNorm(G, eps) over x[N][C][HW], affine w/b (may be NULL), then SiLU
 * when apply_silu: y = mul(t, sigmoid(t)), t = add(mul(norm, w), b). */
void or_groupnorm_silu_f32(const float *x, int64_t N, int64_t C, int64_t HW,
                           int64_t G, const float *w, const float *b, float eps,
                           int apply_silu, float *y, int nthreads);

/* Euler step x + dt * v (FlowMatchEulerDiscreteScheduler::integrate). */
void or_euler_f32(const float *x, const float *v, float dt, int64_t n, float *y);

/* ---- ggml block quantisation ------------------------------------------- */
/* Q8_0: 32-element blocks {fp16 d; int8 qs[32]} = 34 bytes.
 * Q4_K: 256-element super-blocks {fp16 d; fp16 dmin; u8 scales[12];
 *       u8 qs[128]} = 144 bytes. n is the element count. */
void or_quantize_q8_0(const float *x, int64_t n, uint8_t *dst);
void or_dequant_q8_0_f32(const uint8_t *src, int64_t n, float *y, int nthreads);
void or_quantize_q4_K(const float *x, int64_t n, uint8_t *dst);
void or_dequant_q4_K_f32(const uint8_t *src, int64_t n, float *y, int nthreads);
void or_q4_K_scale_min(int j, const uint8_t *scales12, uint8_t *sc, uint8_t *m);

/* ---- small helpers used by the timed CPU baseline ----------------------- */
/* ---- matmul and attention (fp32) --------------------------------------- */
/* y[m][n] = sum_k x[m][k] * w[n][k], then + b[n] when b is given: ggml_mul_mat(w, x)
 * followed by ggml_add, as Linear::forward emits them (src/nn/Linear.cpp:17-36).
 * Each dot product accumulates in double over 4 interleaved lanes (lane l
 * takes k = l mod 4), the lanes are summed in order, and the sum is rounded
 * once to fp32.  Strides are in elements. */
/* conv_2d_direct (stride 1, padding P, square kernel K) + bias, NCHW; up2:
 * on the nearest 2x upscale of x.  See oracle.c. */
void or_conv2d_f32(const float *x, int64_t N, int64_t Ci, int64_t H, int64_t W,
                   const float *w, int64_t Co, int64_t K, int64_t P, const float *b,
                   int up2, float *y, int nthreads);

void or_linear_f32(const float *x, int64_t M, int64_t K, int64_t x_stride,
                   const float *w, int64_t N, int64_t w_stride, const float *b,
                   float *y, int64_t y_stride, int nthreads);
/* ggml's CPU mul_mat for a Q8_0 weight: activation rows quantised to Q8_0,
 * integer block dots, fp32 block sum (see oracle.c).  w: N rows of K/32
 * blocks of 34 bytes; K % 32 == 0. */
void or_linear_q8_0_ggml(const float *x, int64_t M, int64_t K, int64_t x_stride, const uint8_t *w, int64_t N,
                         const float *b, float *y, int64_t y_stride, int nthreads);

/* Unmasked softmax attention, ggml_flash_attn_ext as FlashAttentionOp::operator()
 * calls it (src/nn/attention/FlashAttentionOp.cpp:84-94): for each head h and
 * query s, o = sum_j softmax_j(scale * <q, k_j>) v_j with scores, exponentials
 * and sums in double (max-subtracted), rounded once to fp32.  Element (s, h, d)
 * of q is q[s*q_str[0] + h*q_str[1] + d]; likewise k, v (seq_kv tokens), o. */
void or_attention_f32(const float *q, const float *k, const float *v, float *o,
                      int64_t heads, int64_t seq_q, int64_t seq_kv, int64_t head_dim,
                      const int64_t q_str[2], const int64_t k_str[2], const int64_t v_str[2],
                      const int64_t o_str[2], float scale, int nthreads);

int or_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
