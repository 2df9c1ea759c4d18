/*
 * oracle.c -- the oracle: CPU restatement of ggml CPU-backend semantics for
 * the Flux2 DiT elementwise/reduction chain.  Test infrastructure only; see
 * oracle.h for the rules on who may call it.
 *
 * Every function names the reference call site whose emitted ggml graph it
 * reproduces (paths relative to the reference repository root) and the
 * ggml operator whose published CPU algorithm it restates.  ggml is the
 * reference's un-vendored submodule (https://github.com/ggml-org/ggml,
 * pinned commit unknown); its CPU algorithms are restated from their
 * published description, not copied.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define OR_OMP_THREADS(nt) num_threads((nt) > 0 ? (nt) : or_max_threads())

int or_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ======================================================================== */
/* std::mt19937_64 (the C++11 standard's parameters) + Box-Muller            */
/* ======================================================================== */

typedef struct {
    uint64_t mt[312];
    int idx;
} mt64_t;

static void mt64_seed(mt64_t *s, uint64_t seed) {
    s->mt[0] = seed;
    for (int i = 1; i < 312; ++i)
        s->mt[i] = 6364136223846793005ULL * (s->mt[i - 1] ^ (s->mt[i - 1] >> 62)) + (uint64_t)i;
    s->idx = 312;
}

static uint64_t mt64_next(mt64_t *s) {
    static const uint64_t upper = 0xFFFFFFFF80000000ULL, lower = 0x7FFFFFFFULL;
    if (s->idx >= 312) {
        for (int i = 0; i < 312; ++i) {
            uint64_t y = (s->mt[i] & upper) | (s->mt[(i + 1) % 312] & lower);
            uint64_t v = s->mt[(i + 156) % 312] ^ (y >> 1);
            if (y & 1) v ^= 0xB5026F5AA96619E9ULL;
            s->mt[i] = v;
        }
        s->idx = 0;
    }
    uint64_t x = s->mt[s->idx++];
    x ^= (x >> 29) & 0x5555555555555555ULL;
    x ^= (x << 17) & 0x71D67FFFEDA60000ULL;
    x ^= (x << 37) & 0xFFF7EEE000000000ULL;
    x ^= x >> 43;
    return x;
}

uint64_t or_mt64_nth(uint64_t seed, uint64_t n) {
    mt64_t s;
    uint64_t v = 0;
    mt64_seed(&s, seed);
    for (uint64_t i = 0; i < n; ++i) v = mt64_next(&s);
    return v;
}

/* Box-Muller on 53-bit uniforms: u1 in (0,1], u2 in [0,1); each pair of
 * draws yields (r cos 2πu2, r sin 2πu2), emitted in that order.  Written
 * in-repo because std::normal_distribution is implementation-defined. */
void or_randn_f32(uint64_t seed, int64_t n, float mean, float std, float *out) {
    mt64_t s;
    const double two_pi = 6.283185307179586476925286766559;
    mt64_seed(&s, seed);
    for (int64_t i = 0; i < n; i += 2) {
        double u1 = (double)((mt64_next(&s) >> 11) + 1) * 0x1.0p-53;
        double u2 = (double)(mt64_next(&s) >> 11) * 0x1.0p-53;
        double r = sqrt(-2.0 * log(u1));
        double z0 = r * cos(two_pi * u2), z1 = r * sin(two_pi * u2);
        out[i] = (float)((double)mean + (double)std * z0);
        if (i + 1 < n) out[i + 1] = (float)((double)mean + (double)std * z1);
    }
}

void or_rand_int32(uint64_t seed, int64_t n, int32_t lo, int32_t hi, int32_t *out) {
    mt64_t s;
    uint64_t span = (uint64_t)((int64_t)hi - (int64_t)lo + 1);
    mt64_seed(&s, seed);
    for (int64_t i = 0; i < n; ++i) out[i] = (int32_t)((int64_t)lo + (int64_t)(mt64_next(&s) % span));
}

/* ======================================================================== */
/* hash-drawn test weights                                                   */
/* ======================================================================== */

/* Synthetic Linear and RMSNorm weights whose exact values depend only on
 * integer arithmetic, so a device-side run (dit_cli --hash-weights) and this
 * restatement produce the same bytes with no libm involved.  For a seed and
 * a parameter path (e.g. "transformer_blocks.0.attn.to_q.weight"):
 *   key  = splitmix64(seed * G ^ fnv1a64(path)),  G = 0x9E3779B97F4A7C15
 *   z(i) = splitmix64(key + i * G)
 * Q8_0 block b of a [rows, cols] weight (row-major over rows x cols/32):
 *   d = fp16 bits 0x0E00 | (z(9b) & 0x1FF)  (d in [3.66e-4, 4.88e-4))
 *   code 4(k-1)+m, k = 1..8, m = 0..3: bytes y = z(9b+k) little-endian,
 *   q = (y[2m] + y[2m+1] - 255) / 2, truncated toward zero, in [-127, 127]
 *   (triangular, std 52.2, so d*q has std ~0.022).
 * RMSNorm weight i: 1.0f + (float)((int32)(z(i) >> 40) - 2^23) * 2^-28,
 * one fp32 rounding. */
static const uint64_t or_golden = 0x9E3779B97F4A7C15ULL;

/* splitmix64's output function (Steele, Lea, Flood 2014; Vigna's public
 * splitmix64.c): the n-th output of the generator seeded s is
 * or_splitmix64(s + n * G), n = 1, 2, ... */
uint64_t or_splitmix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

/* 64-bit FNV-1a (offset basis 0xCBF29CE484222325, prime 0x100000001B3). */
uint64_t or_fnv1a64(const char *s) {
    uint64_t h = 0xCBF29CE484222325ULL;
    for (const unsigned char *c = (const unsigned char *)s; *c; ++c) h = (h ^ *c) * 0x100000001B3ULL;
    return h;
}

uint64_t or_hash_key(uint64_t seed, const char *path) { return or_splitmix64(seed * or_golden ^ or_fnv1a64(path)); }

void or_hash_q8_0(uint64_t seed, const char *path, int64_t rows, int64_t cols, uint8_t *dst, int nthreads) {
    const uint64_t key = or_hash_key(seed, path);
    const int64_t nb = rows * (cols / 32);
#pragma omp parallel for schedule(static) OR_OMP_THREADS(nthreads)
    for (int64_t b = 0; b < nb; ++b) {
        uint8_t *blk = dst + b * 34;
        const uint64_t z0 = or_splitmix64(key + (uint64_t)(9 * b) * or_golden);
        const uint16_t d = (uint16_t)(0x0E00u | (uint32_t)(z0 & 0x1FF));
        blk[0] = (uint8_t)(d & 0xFF);
        blk[1] = (uint8_t)(d >> 8);
        for (int k = 1; k <= 8; ++k) {
            const uint64_t z = or_splitmix64(key + (uint64_t)(9 * b + k) * or_golden);
            for (int m = 0; m < 4; ++m) {
                const int y0 = (int)((z >> (16 * m)) & 0xFF), y1 = (int)((z >> (16 * m + 8)) & 0xFF);
                blk[2 + 4 * (k - 1) + m] = (uint8_t)(int8_t)((y0 + y1 - 255) / 2);
            }
        }
    }
}

void or_hash_norm_weight(uint64_t seed, const char *path, int64_t n, float *out) {
    const uint64_t key = or_hash_key(seed, path);
    for (int64_t i = 0; i < n; ++i) {
        const int32_t v = (int32_t)(or_splitmix64(key + (uint64_t)i * or_golden) >> 40) - 8388608;
        out[i] = 1.0f + (float)v * 0x1.0p-28f;
    }
}

/* ======================================================================== */
/* number formats                                                            */
/* ======================================================================== */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    uint32_t e = (h >> 10) & 0x1F, m = h & 0x3FF;
    if (e == 0x1F) return u2f(sign | 0x7F800000u | (m << 13));
    if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in fp32 */
        float v = (float)m * 0x1.0p-24f;
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t or_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
    uint32_t a = x & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) /* inf / nan (nan kept quiet) */
        return sign | 0x7C00 | (a > 0x7F800000u ? (0x200 | ((a >> 13) & 0x3FF)) : 0);
    if (a >= 0x477FF000u) return sign | 0x7C00;        /* rounds to inf */
    if (a < 0x38800000u) {                               /* below 2^-14 */
        uint32_t e = a >> 23;
        if (e < 102) return sign;
        uint32_t mant = (a & 0x7FFFFFu) | 0x800000u;
        uint32_t sh = 126 - e, q = mant >> sh, rem = mant & ((1u << sh) - 1), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (q & 1))) ++q;
        return sign | (uint16_t)q;
    }
    uint32_t r = a - 0x38000000u;
    r = (r + 0xFFFu + ((r >> 13) & 1u)) >> 13;
    return sign | (uint16_t)r;
}

float or_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t or_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 64);
    return (uint16_t)((u + (0x7FFFu + ((u >> 16) & 1u))) >> 16);
}

void or_f32_to_bf16_n(const float *x, int64_t n, uint16_t *y) {
    for (int64_t i = 0; i < n; ++i) y[i] = or_f32_to_bf16(x[i]);
}

void or_bf16_to_f32_n(const uint16_t *x, int64_t n, float *y) {
    for (int64_t i = 0; i < n; ++i) y[i] = or_bf16_to_f32(x[i]);
}

void or_round_bf16_n(const float *x, int64_t n, float *y) {
    for (int64_t i = 0; i < n; ++i) y[i] = or_bf16_to_f32(or_f32_to_bf16(x[i]));
}

/* ======================================================================== */
/* single ggml ops                                                           */
/* ======================================================================== */

/* ggml_norm (CPU): mean and biased variance accumulated in double over the
 * row; y = (x - mean) * 1/sqrtf(var + eps).  Emitted by LayerNorm::forward
 * (src/nn/modules/normalization/LayerNorm.cpp:17) and GroupNorm::forward
 * (src/nn/modules/normalization/GroupNorm.cpp:51-57). */
static void norm_row(const float *x, int64_t n, float eps, float *y) {
    double sum = 0.0;
    for (int64_t i = 0; i < n; ++i) sum += (double)x[i];
    const float mean = (float)(sum / (double)n);
    double sum2 = 0.0;
    for (int64_t i = 0; i < n; ++i) {
        const float v = x[i] - mean;
        y[i] = v;
        sum2 += (double)(v * v);
    }
    const float variance = (float)(sum2 / (double)n);
    const float scale = 1.0f / sqrtf(variance + eps);
    for (int64_t i = 0; i < n; ++i) y[i] *= scale;
}

void or_norm_f32(const float *x, int64_t rows, int64_t cols, float eps, float *y, int nthreads) {
#pragma omp parallel for schedule(static) OR_OMP_THREADS(nthreads)
    for (int64_t r = 0; r < rows; ++r) norm_row(x + r * cols, cols, eps, y + r * cols);
}

/* ggml_rms_norm (CPU): sum of float squares accumulated in double;
 * y = x * 1/sqrtf(mean + eps).  Emitted by RMSNorm::forward
 * (src/nn/modules/normalization/RMSNorm.cpp:13). */
static void rms_norm_row(const float *x, int64_t n, float eps, float *y) {
    double sum = 0.0;
    for (int64_t i = 0; i < n; ++i) sum += (double)(x[i] * x[i]);
    const float mean = (float)(sum / (double)n);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int64_t i = 0; i < n; ++i) y[i] = x[i] * scale;
}

void or_rms_norm_f32(const float *x, int64_t rows, int64_t cols, float eps, float *y, int nthreads) {
#pragma omp parallel for schedule(static) OR_OMP_THREADS(nthreads)
    for (int64_t r = 0; r < rows; ++r) rms_norm_row(x + r * cols, cols, eps, y + r * cols);
}

/* ggml_sigmoid (CPU): 1/(1+expf(-x)).  Emitted by SiLU::forward
 * (src/nn/SiLU.hpp:12). */
static inline float sigmoidf_ggml(float x) { return 1.0f / (1.0f + expf(-x)); }

void or_sigmoid_f32(const float *x, int64_t n, float *y) {
    for (int64_t i = 0; i < n; ++i) y[i] = sigmoidf_ggml(x[i]);
}

/* ggml_scale: y = x * s (Tensor::scale, src/ggml/Tensor.cpp:81-83). */
void or_scale_f32(const float *x, int64_t n, float s, float *y) {
    for (int64_t i = 0; i < n; ++i) y[i] = x[i] * s;
}

/* ggml binary ops: src1 repeats into src0's shape (i1 % ne1 per dim); the
 * operand order is the one Tensor::operator+,-,*,/ picks
 * (src/ggml/Tensor.cpp:97-190). */
void or_binary_f32(int op,
                   const float *a, const int64_t ne_a[4], const int64_t nb_a[4],
                   const float *b, const int64_t ne_b[4], const int64_t nb_b[4],
                   float *dst) {
    int64_t o = 0;
    for (int64_t i3 = 0; i3 < ne_a[3]; ++i3)
    for (int64_t i2 = 0; i2 < ne_a[2]; ++i2)
    for (int64_t i1 = 0; i1 < ne_a[1]; ++i1) {
        const char *ra = (const char *)a + i1 * nb_a[1] + i2 * nb_a[2] + i3 * nb_a[3];
        const char *rb = (const char *)b + (i1 % ne_b[1]) * nb_b[1] + (i2 % ne_b[2]) * nb_b[2]
                                         + (i3 % ne_b[3]) * nb_b[3];
        for (int64_t i0 = 0; i0 < ne_a[0]; ++i0) {
            const float x = *(const float *)(ra + i0 * nb_a[0]);
            const float y = *(const float *)(rb + (i0 % ne_b[0]) * nb_b[0]);
            float r;
            switch (op) {
                case 0: r = x + y; break;
                case 1: r = x - y; break;
                case 2: r = x * y; break;
                default: r = x / y; break;
            }
            dst[o++] = r;
        }
    }
}

/* ggml_concat of two contiguous tensors along ggml dim `dim`
 * (Tensor::cat, src/ggml/Tensor.cpp:252-299). */
void or_concat_f32(const float *a, const int64_t ne_a[4],
                   const float *b, const int64_t ne_b[4], int dim, float *dst) {
    int64_t ne[4];
    for (int d = 0; d < 4; ++d) ne[d] = ne_a[d];
    ne[dim] = ne_a[dim] + ne_b[dim];
    int64_t o = 0;
    for (int64_t i3 = 0; i3 < ne[3]; ++i3)
    for (int64_t i2 = 0; i2 < ne[2]; ++i2)
    for (int64_t i1 = 0; i1 < ne[1]; ++i1)
    for (int64_t i0 = 0; i0 < ne[0]; ++i0) {
        int64_t idx[4] = {i0, i1, i2, i3};
        const float *src = a;
        const int64_t *sne = ne_a;
        if (idx[dim] >= ne_a[dim]) { idx[dim] -= ne_a[dim]; src = b; sne = ne_b; }
        dst[o++] = src[((idx[3] * sne[2] + idx[2]) * sne[1] + idx[1]) * sne[0] + idx[0]];
    }
}

/* ggml_rope_cache_init + rope_yarn with ext_factor == 0: the angle is a
 * float recurrence theta_{i+1} = theta_i * powf(base, -2/n_dims) started at
 * theta_0 = p * freq_scale; cos/sin via libm cosf/sinf, times attn_factor. */
void or_rope_cache(float p, int n_dims, int64_t ne0, float freq_base,
                   float freq_scale, float attn_factor, float *cache) {
    const float theta_scale = powf(freq_base, -2.0f / (float)n_dims);
    float theta = p;
    for (int64_t i0 = 0; i0 < ne0; i0 += 2) {
        const float t = freq_scale * theta;
        cache[i0 + 0] = cosf(t) * attn_factor;
        cache[i0 + 1] = sinf(t) * attn_factor;
        theta *= theta_scale;
    }
}

/* ggml_rope_ext, GGML_ROPE_TYPE_NORMAL: adjacent pairs (x[2i], x[2i+1])
 * rotated by the cached angle of the row's position.  Emitted four times per
 * q/k by Flux2PosEmbed::forward
 * (src/diffusers/models/transformers/flux2/Flux2PosEmbed.hpp:79-95). */
void or_rope_normal_f32(const float *x, const int64_t ne[4], const int64_t nb[4],
                        const int32_t *pos, int n_dims, float freq_base,
                        float freq_scale, float attn_factor, float *dst) {
    float *cache = (float *)malloc(sizeof(float) * (size_t)(ne[0] + 2));
    int64_t o = 0;
    for (int64_t i3 = 0; i3 < ne[3]; ++i3)
    for (int64_t i2 = 0; i2 < ne[2]; ++i2) {
        or_rope_cache((float)pos[i2], n_dims, ne[0], freq_base, freq_scale, attn_factor, cache);
        for (int64_t i1 = 0; i1 < ne[1]; ++i1) {
            const char *row = (const char *)x + i1 * nb[1] + i2 * nb[2] + i3 * nb[3];
            for (int64_t i0 = 0; i0 < ne[0]; i0 += 2) {
                const float x0 = *(const float *)(row + i0 * nb[0]);
                const float x1 = *(const float *)(row + (i0 + 1) * nb[0]);
                if (i0 < n_dims) {
                    const float c = cache[i0], s = cache[i0 + 1];
                    dst[o + i0] = x0 * c - x1 * s;
                    dst[o + i0 + 1] = x0 * s + x1 * c;
                } else {
                    dst[o + i0] = x0;
                    dst[o + i0 + 1] = x1;
                }
            }
            o += ne[0];
        }
    }
    free(cache);
}

/* ======================================================================== */
/* chains                                                                    */
/* ======================================================================== */

/* adaLN: LayerNorm(eps, no affine) then (1 + scale) * n + shift.
 * Reference: Flux2SingleTransformerBlock.hpp:50-54, Flux2TransformerBlock.hpp
 * :63-72 and :91-92, AdaLayerNormContinuous.inl:38-40.  Emitted graph:
 * t = add(scale, 1.0f) [Tensor.hpp:352-355, 403-406]; m = mul(norm(x), t);
 * y = add(m, shift) [operand order from Tensor.cpp:97-120, 148-170]. */
void or_adaln_f32(const float *x, int64_t rows, int64_t cols,
                  const float *shift, const float *scale, float eps, float *y,
                  int nthreads) {
    float *t = (float *)malloc(sizeof(float) * (size_t)cols);
    for (int64_t c = 0; c < cols; ++c) t[c] = scale[c] + 1.0f;
#pragma omp parallel for schedule(static) OR_OMP_THREADS(nthreads)
    for (int64_t r = 0; r < rows; ++r) {
        float *yr = y + r * cols;
        norm_row(x + r * cols, cols, eps, yr);
        for (int64_t c = 0; c < cols; ++c) {
            const float m = yr[c] * t[c];
            yr[c] = m + shift[c];
        }
    }
    free(t);
}

/* QK-RMSNorm + Flux2PosEmbed: y = cat_a rope_a(rms_norm(x) * w).
 * Reference: RMSNorm::forward (RMSNorm.cpp:12-22) on the unflattened q/k
 * (Flux2Attention.hpp:93-112, Flux2ParallelSelfAttention.hpp:63-76), then
 * Flux2PosEmbed::forward (Flux2PosEmbed.hpp:29-108): for axis a the dims
 * [a*axis_dim, (a+1)*axis_dim) go through rope_ext with n_dims = axis_dim
 * and position column a, and the sections are concatenated back. */
void or_qk_rmsnorm_rope_f32(const float *x, int64_t tokens, int64_t heads,
                            int64_t head_dim, const float *w, float eps,
                            const int32_t *pos, int64_t pos_stride, int n_axes,
                            int axis_dim, float freq_base, float *y, int nthreads) {
#pragma omp parallel OR_OMP_THREADS(nthreads)
    {
        float *z = (float *)malloc(sizeof(float) * (size_t)head_dim);
        float *cache = (float *)malloc(sizeof(float) * (size_t)(axis_dim + 2) * (size_t)n_axes);
#pragma omp for schedule(static)
        for (int64_t s = 0; s < tokens; ++s) {
            for (int a = 0; a < n_axes; ++a)
                or_rope_cache((float)pos[s * pos_stride + a], axis_dim, axis_dim, freq_base,
                              1.0f, 1.0f, cache + (int64_t)a * (axis_dim + 2));
            for (int64_t h = 0; h < heads; ++h) {
                const float *xr = x + (s * heads + h) * head_dim;
                float *yr = y + (s * heads + h) * head_dim;
                rms_norm_row(xr, head_dim, eps, z);
                for (int64_t d = 0; d < head_dim; ++d) z[d] = z[d] * w[d];
                for (int a = 0; a < n_axes; ++a) {
                    const float *ca = cache + (int64_t)a * (axis_dim + 2);
                    const int64_t base = (int64_t)a * axis_dim;
                    for (int i0 = 0; i0 < axis_dim; i0 += 2) {
                        const float x0 = z[base + i0], x1 = z[base + i0 + 1];
                        const float c = ca[i0], sn = ca[i0 + 1];
                        yr[base + i0] = x0 * c - x1 * sn;
                        yr[base + i0 + 1] = x0 * sn + x1 * c;
                    }
                }
                for (int64_t d = (int64_t)n_axes * axis_dim; d < head_dim; ++d) yr[d] = z[d];
            }
        }
        free(z);
        free(cache);
    }
}

/* Flux2SwiGLU::forward (Flux2SwiGLU.hpp:17-21) with SiLU = x*sigmoid(x)
 * (SiLU.hpp:12): s = sigmoid(g); a = mul(g, s); y = mul(a, u). */
void or_swiglu_f32(const float *g, int64_t g_stride, const float *u, int64_t u_stride,
                   int64_t rows, int64_t cols, float *y, int nthreads) {
#pragma omp parallel for schedule(static) OR_OMP_THREADS(nthreads)
    for (int64_t r = 0; r < rows; ++r) {
        const float *gr = g + r * g_stride, *ur = u + r * u_stride;
        float *yr = y + r * cols;
        for (int64_t c = 0; c < cols; ++c) {
            const float s = sigmoidf_ggml(gr[c]);
            const float a = gr[c] * s;
            yr[c] = a * ur[c];
        }
    }
}

/* Gated residual h + gate * o (Flux2SingleTransformerBlock.hpp:58,
 * Flux2TransformerBlock.hpp:86-87, 97, 100-101, 111): t = mul(o, gate)
 * [gate is the smaller operand, so it goes second], y = add(h, t). */
void or_gated_residual_f32(const float *h, const float *o, const float *gate,
                           int64_t rows, int64_t cols, float *y, int nthreads) {
#pragma omp parallel for schedule(static) OR_OMP_THREADS(nthreads)
    for (int64_t r = 0; r < rows; ++r) {
        const float *hr = h + r * cols, *or_ = o + r * cols;
        float *yr = y + r * cols;
        for (int64_t c = 0; c < cols; ++c) {
            const float t = or_[c] * gate[c];
            yr[c] = hr[c] + t;
        }
    }
}

/* GroupNorm::forward (GroupNorm.cpp:25-108): reshape [N, G, C/G*HW], norm
 * per (n, g) row, reshape back, mul(x, w[1,C,1,1]), add(., b[1,C,1,1]);
 * followed by SiLU::forward (SiLU.hpp:12) as in ResnetBlock2D.inl:111-122,
 * 160-171 and Decoder.hpp:147-160. */
void or_groupnorm_silu_f32(const float *x, int64_t N, int64_t C, int64_t HW,
                           int64_t G, const float *w, const float *b, float eps,
                           int apply_silu, float *y, int nthreads) {
    const int64_t cg = C / G, len = cg * HW;
#pragma omp parallel for schedule(dynamic, 1) OR_OMP_THREADS(nthreads)
    for (int64_t ng = 0; ng < N * G; ++ng) {
        const int64_t n = ng / G, g = ng % G;
        const float *xr = x + (n * C + g * cg) * HW;
        float *yr = y + (n * C + g * cg) * HW;
        norm_row(xr, len, eps, yr);
        for (int64_t cc = 0; cc < cg; ++cc) {
            const int64_t c = g * cg + cc;
            float *yc = yr + cc * HW;
            for (int64_t i = 0; i < HW; ++i) {
                float t = yc[i];
                if (w) t = t * w[c];
                if (b) t = t + b[c];
                if (apply_silu) {
                    const float s = sigmoidf_ggml(t);
                    t = t * s;
                }
                yc[i] = t;
            }
        }
    }
}

/* FlowMatchEulerDiscreteScheduler::integrate (.cpp:210-222):
 * sample + dt * v -> t = mul(v, dt) [dt is the [1] operand], add(x, t). */
void or_euler_f32(const float *x, const float *v, float dt, int64_t n, float *y) {
    for (int64_t i = 0; i < n; ++i) {
        const float t = v[i] * dt;
        y[i] = x[i] + t;
    }
}

/* ======================================================================== */
/* ggml block quantisation                                                   */
/* ======================================================================== */

/* Q8_0 reference quantiser: d = amax/127 (stored fp16), q = roundf(x/d). */
void or_quantize_q8_0(const float *x, int64_t n, uint8_t *dst) {
    for (int64_t blk = 0; blk < n / 32; ++blk) {
        const float *xb = x + blk * 32;
        uint8_t *o = dst + blk * 34;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(xb[j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t dh = or_f32_to_f16(d);
        memcpy(o, &dh, 2);
        for (int j = 0; j < 32; ++j) o[2 + j] = (uint8_t)(int8_t)roundf(xb[j] * id);
    }
}

/* Q8_0 dequantisation: y = fp16_to_fp32(d) * q, one IEEE rounding. */
void or_dequant_q8_0_f32(const uint8_t *src, int64_t n, float *y, int nthreads) {
#pragma omp parallel for schedule(static) OR_OMP_THREADS(nthreads)
    for (int64_t blk = 0; blk < n / 32; ++blk) {
        const uint8_t *b = src + blk * 34;
        uint16_t dh;
        memcpy(&dh, b, 2);
        const float d = or_f16_to_f32(dh);
        for (int j = 0; j < 32; ++j) y[blk * 32 + j] = d * (float)(int8_t)b[2 + j];
    }
}

/* Q4_K 6-bit (scale, min) unpack for sub-block j (0..7) of a super-block:
 * j < 4: low 6 bits of bytes j and j+4; j >= 4: the nibbles of byte j+4
 * joined with the top two bits of bytes j-4 (scale) and j (min). */
void or_q4_K_scale_min(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* Q4_K dequantisation: within each 64-element chunk c the low nibbles of
 * qs[32c .. 32c+32) give elements [64c, 64c+32) with sub-block 2c, the high
 * nibbles give [64c+32, 64c+64) with sub-block 2c+1;
 * y = (d * sc) * q - (dmin * m), each product and the difference rounded. */
void or_dequant_q4_K_f32(const uint8_t *src, int64_t n, float *y, int nthreads) {
#pragma omp parallel for schedule(static) OR_OMP_THREADS(nthreads)
    for (int64_t blk = 0; blk < n / 256; ++blk) {
        const uint8_t *b = src + blk * 144;
        uint16_t dh, mh;
        memcpy(&dh, b, 2);
        memcpy(&mh, b + 2, 2);
        const float d = or_f16_to_f32(dh), dmin = or_f16_to_f32(mh);
        const uint8_t *scales = b + 4, *qs = b + 16;
        float *yb = y + blk * 256;
        for (int c = 0; c < 4; ++c) {
            uint8_t sc, m;
            or_q4_K_scale_min(2 * c, scales, &sc, &m);
            const float d1 = d * (float)sc, m1 = dmin * (float)m;
            or_q4_K_scale_min(2 * c + 1, scales, &sc, &m);
            const float d2 = d * (float)sc, m2 = dmin * (float)m;
            for (int l = 0; l < 32; ++l) {
                const float p1 = d1 * (float)(qs[32 * c + l] & 0x0F);
                yb[64 * c + l] = p1 - m1;
                const float p2 = d2 * (float)(qs[32 * c + l] >> 4);
                yb[64 * c + 32 + l] = p2 - m2;
            }
        }
    }
}

static inline int nearest_int_rne(float v) { return (int)lrintf(v); }

/* ggml's make_qkx2_quants: weighted asymmetric 4-bit fit of one 32-element
 * sub-block, searching nstep+1 candidate inverse scales around the
 * min/max-based one and refitting (scale, min) by weighted least squares. */
static float fit_q4_subblock(const float *x, const float *wt, uint8_t *L, float *the_min,
                             uint8_t *Laux) {
    const int n = 32, nmax = 15, nstep = 20;
    const float rmin = -1.0f, rdelta = 0.1f;
    float lo = x[0], hi = x[0], sum_w = wt[0], sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < lo) lo = x[i];
        if (x[i] > hi) hi = x[i];
        sum_w += wt[i];
        sum_x += wt[i] * x[i];
    }
    if (lo > 0) lo = 0;
    if (hi == lo) {
        memset(L, 0, (size_t)n);
        *the_min = -lo;
        return 0.0f;
    }
    float iscale = nmax / (hi - lo), scale = 1.0f / iscale, best = 0.0f;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int_rne(iscale * (x[i] - lo));
        l = l < 0 ? 0 : (l > nmax ? nmax : l);
        L[i] = (uint8_t)l;
        const float diff = scale * L[i] + lo - x[i];
        best += wt[i] * (diff * diff);
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (hi - lo);
        float sl = 0, sl2 = 0, sxl = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int_rne(iscale * (x[i] - lo));
            l = l < 0 ? 0 : (l > nmax ? nmax : l);
            Laux[i] = (uint8_t)l;
            sl += wt[i] * l;
            sl2 += wt[i] * l * l;
            sxl += wt[i] * l * x[i];
        }
        const float D = sum_w * sl2 - sl * sl;
        if (D > 0) {
            float s_ = (sum_w * sxl - sum_x * sl) / D;
            float m_ = (sl2 * sum_x - sl * sxl) / D;
            if (m_ > 0) {
                m_ = 0;
                s_ = sxl / sl2;
            }
            float err = 0;
            for (int i = 0; i < n; ++i) {
                const float diff = s_ * Laux[i] + m_ - x[i];
                err += wt[i] * (diff * diff);
            }
            if (err < best) {
                memcpy(L, Laux, (size_t)n);
                best = err;
                scale = s_;
                lo = m_;
            }
        }
    }
    *the_min = -lo;
    return scale;
}

/* ggml's reference Q4_K quantiser (quantize_row_q4_K_ref): per sub-block
 * fit, 6-bit quantisation of scales and mins against the super-block
 * maxima, then the final 4-bit codes recomputed from the stored values. */
void or_quantize_q4_K(const float *x, int64_t n, uint8_t *dst) {
    uint8_t L[256], Laux[32];
    float wt[32], mins[8], scales[8];
    for (int64_t blk = 0; blk < n / 256; ++blk) {
        const float *xb = x + blk * 256;
        uint8_t *o = dst + blk * 144;
        uint8_t *sc12 = o + 4, *qs = o + 16;
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < 8; ++j) {
            float sum_x2 = 0;
            for (int l = 0; l < 32; ++l) sum_x2 += xb[32 * j + l] * xb[32 * j + l];
            const float av_x = sqrtf(sum_x2 / 32);
            for (int l = 0; l < 32; ++l) wt[l] = av_x + fabsf(xb[32 * j + l]);
            scales[j] = fit_q4_subblock(xb + 32 * j, wt, L + 32 * j, &mins[j], Laux);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
        const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
        memset(sc12, 0, 12);
        for (int j = 0; j < 8; ++j) {
            uint8_t ls = (uint8_t)nearest_int_rne(inv_scale * scales[j]);
            uint8_t lm = (uint8_t)nearest_int_rne(inv_min * mins[j]);
            if (ls > 63) ls = 63;
            if (lm > 63) lm = 63;
            if (j < 4) {
                sc12[j] = ls;
                sc12[j + 4] = lm;
            } else {
                sc12[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
                sc12[j - 4] |= (uint8_t)((ls >> 4) << 6);
                sc12[j] |= (uint8_t)((lm >> 4) << 6);
            }
        }
        const uint16_t dh = or_f32_to_f16(max_scale / 63.f), mh = or_f32_to_f16(max_min / 63.f);
        memcpy(o, &dh, 2);
        memcpy(o + 2, &mh, 2);
        for (int j = 0; j < 8; ++j) {
            uint8_t sc, m;
            or_q4_K_scale_min(j, sc12, &sc, &m);
            const float d = or_f16_to_f32(dh) * sc;
            if (d == 0.0f) continue;
            const float dm = or_f16_to_f32(mh) * m;
            for (int ii = 0; ii < 32; ++ii) {
                int l = nearest_int_rne((xb[32 * j + ii] + dm) / d);
                L[32 * j + ii] = (uint8_t)(l < 0 ? 0 : (l > 15 ? 15 : l));
            }
        }
        for (int c = 0; c < 4; ++c)
            for (int l = 0; l < 32; ++l)
                qs[32 * c + l] = (uint8_t)(L[64 * c + l] | (L[64 * c + 32 + l] << 4));
    }
}

/* ======================================================================== */
/* matmul and attention                                                     */
/* ======================================================================== */

typedef double or_v4d __attribute__((vector_size(32)));

static inline or_v4d or_load4d(const float *p) {
    or_v4d r = {(double)p[0], (double)p[1], (double)p[2], (double)p[3]};
    return r;
}

static inline double or_hsum4d(or_v4d a) { return ((a[0] + a[1]) + a[2]) + a[3]; }

/* One dot product in the lane order documented in oracle.h. */
static double or_dot_lanes(const float *a, const float *b, int64_t K) {
    or_v4d acc = {0, 0, 0, 0};
    int64_t k = 0;
    for (; k + 4 <= K; k += 4) acc += or_load4d(a + k) * or_load4d(b + k);
    for (; k < K; ++k) acc[k & 3] += (double)a[k] * (double)b[k];
    return or_hsum4d(acc);
}

/* ggml_mul_mat(w, x) + ggml_add(b): src/nn/Linear.cpp:17-36.  Blocked 2x4
 * over (x rows, w rows) so each loaded vector serves several dot products;
 * every dot product keeps the lane order of or_dot_lanes. */
void or_linear_f32(const float *x, int64_t M, int64_t K, int64_t x_stride,
                   const float *w, int64_t N, int64_t w_stride, const float *b,
                   float *y, int64_t y_stride, int nthreads) {
    enum { MB = 32, NB = 64 };
    const int64_t nblk = (N + NB - 1) / NB;
#pragma omp parallel for schedule(dynamic, 1) OR_OMP_THREADS(nthreads)
    for (int64_t jb = 0; jb < nblk; ++jb) {
        const int64_t j0 = jb * NB, j1 = j0 + NB < N ? j0 + NB : N;
        for (int64_t i0 = 0; i0 < M; i0 += MB) {
            const int64_t i1 = i0 + MB < M ? i0 + MB : M;
            for (int64_t i = i0; i < i1; i += 2) {
                for (int64_t j = j0; j < j1; j += 4) {
                    if (i + 2 > i1 || j + 4 > j1 || (K & 3)) {
                        for (int64_t ii = i; ii < i1 && ii < i + 2; ++ii)
                            for (int64_t jj = j; jj < j1 && jj < j + 4; ++jj)
                                y[ii * y_stride + jj] =
                                    (float)or_dot_lanes(x + ii * x_stride, w + jj * w_stride, K);
                        continue;
                    }
                    const float *x0 = x + i * x_stride, *x1 = x0 + x_stride;
                    const float *w0 = w + j * w_stride, *w1 = w0 + w_stride, *w2 = w1 + w_stride,
                                *w3 = w2 + w_stride;
                    or_v4d a00 = {0, 0, 0, 0}, a01 = a00, a02 = a00, a03 = a00;
                    or_v4d a10 = a00, a11 = a00, a12 = a00, a13 = a00;
                    for (int64_t k = 0; k < K; k += 4) {
                        const or_v4d p0 = or_load4d(x0 + k), p1 = or_load4d(x1 + k);
                        const or_v4d q0 = or_load4d(w0 + k), q1 = or_load4d(w1 + k),
                                     q2 = or_load4d(w2 + k), q3 = or_load4d(w3 + k);
                        a00 += p0 * q0; a01 += p0 * q1; a02 += p0 * q2; a03 += p0 * q3;
                        a10 += p1 * q0; a11 += p1 * q1; a12 += p1 * q2; a13 += p1 * q3;
                    }
                    float *y0 = y + i * y_stride + j, *y1 = y0 + y_stride;
                    y0[0] = (float)or_hsum4d(a00); y0[1] = (float)or_hsum4d(a01);
                    y0[2] = (float)or_hsum4d(a02); y0[3] = (float)or_hsum4d(a03);
                    y1[0] = (float)or_hsum4d(a10); y1[1] = (float)or_hsum4d(a11);
                    y1[2] = (float)or_hsum4d(a12); y1[3] = (float)or_hsum4d(a13);
                }
            }
        }
        if (b)
            for (int64_t i = 0; i < M; ++i)
                for (int64_t j = j0; j < j1; ++j) y[i * y_stride + j] = y[i * y_stride + j] + b[j];
    }
}

/* ggml's CPU mul_mat for a Q8_0 weight (Linear::forward -> Runtime::mul_mat,
 * src/nn/Linear.cpp:17-36, on the reference's Q8_0 checkpoints), restated
 * from public ggml (the submodule is not vendored, so its pinned commit is
 * unknown): Q8_0's vec_dot type is Q8_0, so every activation row is first
 * quantised to Q8_0 blocks by the rule of or_quantize_q8_0, then
 *   y[i][j] = sum over blocks b, in order, of
 *             (float)(sum_t qx[t] * qw[t]) * (fp16(d_x) * fp16(d_w))
 * with the 32-term integer dot exact and each block term and the running sum
 * rounded to fp32 (ggml_vec_dot_q8_0_q8_0's scalar form; its SIMD forms
 * regroup the same fp32 sum).  w: N rows of K/32 blocks of 34 bytes. */
void or_linear_q8_0_ggml(const float *x, int64_t M, int64_t K, int64_t x_stride, const uint8_t *w, int64_t N,
                         const float *b, float *y, int64_t y_stride, int nthreads) {
    const int64_t nb = K / 32, rb = nb * 34;
    int8_t *qx = (int8_t *)malloc((size_t)(M * K));
    float *dx = (float *)malloc((size_t)(M * nb) * sizeof(float));
    int8_t *qw = (int8_t *)malloc((size_t)(N * K));
    float *dw = (float *)malloc((size_t)(N * nb) * sizeof(float));
#pragma omp parallel for schedule(static) OR_OMP_THREADS(nthreads)
    for (int64_t i = 0; i < M; ++i) {
        uint8_t blk[34];
        for (int64_t c = 0; c < nb; ++c) {
            or_quantize_q8_0(x + i * x_stride + c * 32, 32, blk);
            uint16_t dh;
            memcpy(&dh, blk, 2);
            dx[i * nb + c] = or_f16_to_f32(dh);
            memcpy(qx + i * K + c * 32, blk + 2, 32);
        }
    }
#pragma omp parallel for schedule(static) OR_OMP_THREADS(nthreads)
    for (int64_t j = 0; j < N; ++j)
        for (int64_t c = 0; c < nb; ++c) {
            const uint8_t *blk = w + j * rb + c * 34;
            uint16_t dh;
            memcpy(&dh, blk, 2);
            dw[j * nb + c] = or_f16_to_f32(dh);
            memcpy(qw + j * K + c * 32, blk + 2, 32);
        }
    enum { JB = 16 };
#pragma omp parallel for schedule(dynamic, 1) OR_OMP_THREADS(nthreads)
    for (int64_t j0 = 0; j0 < N; j0 += JB) {
        const int64_t j1 = j0 + JB < N ? j0 + JB : N;
        for (int64_t i = 0; i < M; ++i) {
            const int8_t *xr = qx + i * K;
            const float *dxr = dx + i * nb;
            for (int64_t j = j0; j < j1; ++j) {
                const int8_t *wr = qw + j * K;
                const float *dwr = dw + j * nb;
                float sum = 0.0f;
                for (int64_t c = 0; c < nb; ++c) {
                    int32_t si = 0;
                    for (int t = 0; t < 32; ++t) si += (int32_t)xr[c * 32 + t] * (int32_t)wr[c * 32 + t];
                    const float term = (float)si * (dxr[c] * dwr[c]);
                    sum = sum + term;
                }
                y[i * y_stride + j] = b ? sum + b[j] : sum;
            }
        }
    }
    free(qx);
    free(dx);
    free(qw);
    free(dw);
}

/* ggml_flash_attn_ext without mask: src/nn/attention/FlashAttentionOp.cpp:84-94. */
void or_attention_f32(const float *q, const float *k, const float *v, float *o,
                      int64_t heads, int64_t seq_q, int64_t seq_kv, int64_t head_dim,
                      const int64_t q_str[2], const int64_t k_str[2], const int64_t v_str[2],
                      const int64_t o_str[2], float scale, int nthreads) {
    const int64_t total = heads * seq_q;
#pragma omp parallel OR_OMP_THREADS(nthreads)
    {
        double *sc = (double *)malloc(sizeof(double) * (size_t)(seq_kv > 0 ? seq_kv : 1));
        double *acc = (double *)malloc(sizeof(double) * (size_t)(head_dim > 0 ? head_dim : 1));
#pragma omp for schedule(static)
        for (int64_t t = 0; t < total; ++t) {
            const int64_t h = t / seq_q, s = t % seq_q;
            const float *qr = q + s * q_str[0] + h * q_str[1];
            double mx = -INFINITY;
            for (int64_t j = 0; j < seq_kv; ++j) {
                sc[j] = or_dot_lanes(qr, k + j * k_str[0] + h * k_str[1], head_dim) * (double)scale;
                if (sc[j] > mx) mx = sc[j];
            }
            double sum = 0.0;
            for (int64_t j = 0; j < seq_kv; ++j) {
                sc[j] = exp(sc[j] - mx);
                sum += sc[j];
            }
            for (int64_t d = 0; d < head_dim; ++d) acc[d] = 0.0;
            for (int64_t j = 0; j < seq_kv; ++j) {
                const float *vr = v + j * v_str[0] + h * v_str[1];
                const double p = sc[j];
                for (int64_t d = 0; d < head_dim; ++d) acc[d] += p * (double)vr[d];
            }
            float *orow = o + s * o_str[0] + h * o_str[1];
            for (int64_t d = 0; d < head_dim; ++d) orow[d] = (float)(acc[d] / sum);
        }
        free(sc);
        free(acc);
    }
}

/* ======================================================================== */
/* conv2d                                                                   */
/* ======================================================================== */

/* ggml_conv_2d_direct(w, x, 1, 1, P, P, 1, 1) followed by the bias ADD of
 * Conv2d::forward (src/nn/modules/conv/Conv2d.cpp:37-108), NCHW, square
 * kernel K; with up2 the input is first the nearest 2x upscale of x, the
 * `upscale(x, 2, NEAREST)` of Upsample2D::forward (Upsample2D.cpp:36-63):
 * xs[n][c][i][j] = x[n][c][i/2][j/2].  Each output is one fp64 sum over
 * (ci, kh, kw) in that order, rounded to fp32, then + b[co] in fp32 (the
 * separate ADD node).  Out-of-image taps read zero. */
void or_conv2d_f32(const float *x, int64_t N, int64_t Ci, int64_t H, int64_t W,
                   const float *w, int64_t Co, int64_t K, int64_t P, const float *b,
                   int up2, float *y, int nthreads) {
    const int64_t Hs = up2 ? 2 * H : H, Ws = up2 ? 2 * W : W;
    const int64_t OH = Hs + 2 * P - K + 1, OW = Ws + 2 * P - K + 1;
#pragma omp parallel for collapse(2) schedule(dynamic, 1) OR_OMP_THREADS(nthreads)
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t co = 0; co < Co; ++co) {
            const float *wc = w + co * Ci * K * K;
            float *yc = y + (n * Co + co) * OH * OW;
            for (int64_t oh = 0; oh < OH; ++oh) {
                for (int64_t ow = 0; ow < OW; ++ow) {
                    double acc = 0.0;
                    for (int64_t ci = 0; ci < Ci; ++ci) {
                        const float *xp = x + (n * Ci + ci) * H * W;
                        for (int64_t kh = 0; kh < K; ++kh) {
                            const int64_t ih = oh + kh - P;
                            if (ih < 0 || ih >= Hs) continue;
                            for (int64_t kw = 0; kw < K; ++kw) {
                                const int64_t iw = ow + kw - P;
                                if (iw < 0 || iw >= Ws) continue;
                                const float xv = up2 ? xp[(ih / 2) * W + iw / 2] : xp[ih * W + iw];
                                acc += (double)wc[(ci * K + kh) * K + kw] * (double)xv;
                            }
                        }
                    }
                    float v = (float)acc;
                    if (b) v = v + b[co];
                    yc[oh * OW + ow] = v;
                }
            }
        }
    }
}

