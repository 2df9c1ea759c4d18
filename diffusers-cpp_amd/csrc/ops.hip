// ops.hip -- unfused single-op kernels with ggml semantics on strided
// ggml-shaped descriptors: the per-op path the graph executor falls back to
// when a node is not part of a fused chain.  Semantics follow the ggml CPU
// ops the reference's Runtime forwards to (src/ggml/ExecutionRuntime.cpp:
// 393-766): binary ops broadcast src1 into src0's shape, norms reduce over
// ne[0], RoPE NORMAL rotates adjacent pairs of the first n_dims elements.
// Element types F32 / F16 / BF16 are read and written through a per-element
// switch; arithmetic is fp32.
#include <math.h>

#include "capi_util.hpp"
#include "common.hpp"

namespace dit {
namespace {

constexpr int kBlock = 256;

struct Desc {
    const char* data;
    int64_t ne[4];
    int64_t nb[4];
    int type;
};

Desc desc_of(const dt_tensor* t) {
    Desc d;
    d.data = (const char*)t->data;
    for (int i = 0; i < 4; ++i) {
        d.ne[i] = t->ne[i];
        d.nb[i] = t->nb[i];
    }
    d.type = t->type;
    return d;
}

__device__ __forceinline__ float ld(const char* p, int type) {
    if (type == DT_TYPE_F32) return *(const float*)p;
    const uint32_t h = *(const uint16_t*)p;
    if (type == DT_TYPE_BF16) return __uint_as_float(h << 16);
    return f16_bits_to_f32(h);
}

__device__ __forceinline__ void st(char* p, int type, float v) {
    if (type == DT_TYPE_F32) *(float*)p = v;
    else if (type == DT_TYPE_BF16) *(uint16_t*)p = (uint16_t)f32_to_bf16_bits(v);
    else *(uint16_t*)p = f32_to_f16_bits(v);
}

__device__ __forceinline__ void unravel(int64_t i, const int64_t* ne, int64_t* idx) {
    idx[0] = i % ne[0];
    i /= ne[0];
    idx[1] = i % ne[1];
    i /= ne[1];
    idx[2] = i % ne[2];
    idx[3] = i / ne[2];
}

__device__ __forceinline__ int64_t offset(const int64_t* idx, const int64_t* nb) {
    return idx[0] * nb[0] + idx[1] * nb[1] + idx[2] * nb[2] + idx[3] * nb[3];
}

__global__ __launch_bounds__(kBlock) void binary_kernel(int op, Desc a, Desc b, Desc d, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        int64_t idx[4], bi[4];
        unravel(i, d.ne, idx);
        for (int k = 0; k < 4; ++k) bi[k] = idx[k] % b.ne[k];
        const float x = ld(a.data + offset(idx, a.nb), a.type);
        const float y = ld(b.data + offset(bi, b.nb), b.type);
        float r;
        switch (op) {
            case DT_BIN_ADD: r = add_rn(x, y); break;
            case DT_BIN_SUB: r = sub_rn(x, y); break;
            case DT_BIN_MUL: r = mul_rn(x, y); break;
            default: r = __fdiv_rn(x, y); break;
        }
        st((char*)d.data + offset(idx, d.nb), d.type, r);
    }
}

__global__ __launch_bounds__(kBlock) void unary_kernel(int op, Desc a, Desc d, float p0, float p1,
                                                       int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        int64_t idx[4];
        unravel(i, d.ne, idx);
        const float x = op == DT_UN_FILL ? 0.0f : ld(a.data + offset(idx, a.nb), a.type);
        float r;
        switch (op) {
            case DT_UN_SIGMOID: r = sigmoid_ref(x); break;
            case DT_UN_EXP: r = expf(x); break;
            case DT_UN_LOG: r = logf(x); break;
            case DT_UN_SQRT: r = sqrtf(x); break;
            case DT_UN_SIN: r = sinf(x); break;
            case DT_UN_COS: r = cosf(x); break;
            case DT_UN_SCALE: r = mul_rn(x, p0); break;
            case DT_UN_CLAMP: r = fminf(fmaxf(x, p0), p1); break;
            case DT_UN_SILU: r = mul_rn(x, sigmoid_ref(x)); break;
            default: r = p0; break;  // FILL
        }
        st((char*)d.data + offset(idx, d.nb), d.type, r);
    }
}

// One block per row of ne[0] elements; rms = false: ggml_norm, true: ggml_rms_norm.
__global__ __launch_bounds__(kBlock) void norm_kernel(Desc a, Desc d, float eps, int rms) {
    __shared__ float red[kBlock / kWave];
    const int64_t row = blockIdx.x;
    int64_t idx[4] = {0, row % a.ne[1], (row / a.ne[1]) % a.ne[2], row / (a.ne[1] * a.ne[2])};
    const char* ar = a.data + offset(idx, a.nb);
    char* dr = (char*)d.data + offset(idx, d.nb);
    const int64_t n = a.ne[0];
    float mean = 0.f;
    if (!rms) {
        float s = 0.f;
        for (int64_t i = threadIdx.x; i < n; i += kBlock) s += ld(ar + i * a.nb[0], a.type);
        mean = block_sum_f32(s, red) / (float)n;
    }
    float s2 = 0.f;
    for (int64_t i = threadIdx.x; i < n; i += kBlock) {
        const float v = ld(ar + i * a.nb[0], a.type) - mean;
        s2 += v * v;
    }
    const float scale = 1.0f / sqrtf(block_sum_f32(s2, red) / (float)n + eps);
    for (int64_t i = threadIdx.x; i < n; i += kBlock) {
        const float v = sub_rn(ld(ar + i * a.nb[0], a.type), mean);
        st(dr + i * d.nb[0], d.type, mul_rn(v, scale));
    }
}

// One thread per adjacent pair (x[2i], x[2i+1]) of a row.
__global__ __launch_bounds__(kBlock) void rope_kernel(Desc a, Desc d, const int32_t* __restrict__ pos,
                                                      int n_dims, float theta_scale, float freq_scale,
                                                      float attn_factor, int64_t n_pairs) {
    const int64_t half = a.ne[0] / 2;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_pairs;
         i += (int64_t)gridDim.x * blockDim.x) {
        int64_t idx[4];
        const int64_t pair = i % half;
        int64_t r = i / half;
        idx[0] = 2 * pair;
        idx[1] = r % a.ne[1];
        r /= a.ne[1];
        idx[2] = r % a.ne[2];
        idx[3] = r / a.ne[2];
        const char* src = a.data + offset(idx, a.nb);
        char* dst = (char*)d.data + offset(idx, d.nb);
        const float x0 = ld(src, a.type), x1 = ld(src + a.nb[0], a.type);
        if (idx[0] < n_dims) {
            float theta = (float)pos[idx[2]];
            for (int64_t k = 0; k < pair; ++k) theta = mul_rn(theta, theta_scale);
            const float t = mul_rn(freq_scale, theta);
            const float c = mul_rn(cosf(t), attn_factor), s = mul_rn(sinf(t), attn_factor);
            st(dst, d.type, sub_rn(mul_rn(x0, c), mul_rn(x1, s)));
            st(dst + d.nb[0], d.type, add_rn(mul_rn(x0, s), mul_rn(x1, c)));
        } else {
            st(dst, d.type, x0);
            st(dst + d.nb[0], d.type, x1);
        }
    }
}

__global__ __launch_bounds__(kBlock) void concat_kernel(Desc a, Desc b, Desc d, int dim, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        int64_t idx[4];
        unravel(i, d.ne, idx);
        const int64_t di = offset(idx, d.nb);
        float v;
        if (idx[dim] < a.ne[dim]) {
            v = ld(a.data + offset(idx, a.nb), a.type);
        } else {
            idx[dim] -= a.ne[dim];
            v = ld(b.data + offset(idx, b.nb), b.type);
        }
        st((char*)d.data + di, d.type, v);
    }
}

__global__ __launch_bounds__(kBlock) void cpy_kernel(Desc a, Desc d, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        int64_t ia[4], id[4];
        unravel(i, a.ne, ia);
        unravel(i, d.ne, id);
        st((char*)d.data + offset(id, d.nb), d.type, ld(a.data + offset(ia, a.nb), a.type));
    }
}

// Same-type element copy by bytes (any 2- or 4-byte type, I32 included).
__global__ __launch_bounds__(kBlock) void concat_raw_kernel(Desc a, Desc b, Desc d, int dim,
                                                            int es, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        int64_t idx[4];
        unravel(i, d.ne, idx);
        char* dst = (char*)d.data + offset(idx, d.nb);
        const char* src;
        if (idx[dim] < a.ne[dim]) {
            src = a.data + offset(idx, a.nb);
        } else {
            idx[dim] -= a.ne[dim];
            src = b.data + offset(idx, b.nb);
        }
        if (es == 4) *(uint32_t*)dst = *(const uint32_t*)src;
        else *(uint16_t*)dst = *(const uint16_t*)src;
    }
}

// Same-type concat of dense tensors whose runs are whole 16-byte vectors:
// d is `rows` runs of (ca + cb) vectors, a's run then b's (the dims above
// `dim` index the runs).  Non-temporal 16-byte copies.
__global__ __launch_bounds__(kBlock) void concat_dense16_kernel(const uint4* __restrict__ a, const uint4* __restrict__ b,
                                                                uint4* __restrict__ d, int64_t ca, int64_t cb,
                                                                int64_t n) {
    const int64_t run = ca + cb;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = i / run, off = i - row * run;
        st_stream(d + i, off < ca ? ld_stream(a + row * ca + off) : ld_stream(b + row * cb + (off - ca)));
    }
}

__global__ __launch_bounds__(kBlock) void cpy_raw_kernel(Desc a, Desc d, int es, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        int64_t ia[4], id[4];
        unravel(i, a.ne, ia);
        unravel(i, d.ne, id);
        const char* src = a.data + offset(ia, a.nb);
        char* dst = (char*)d.data + offset(id, d.nb);
        if (es == 4) *(uint32_t*)dst = *(const uint32_t*)src;
        else *(uint16_t*)dst = *(const uint16_t*)src;
    }
}

unsigned blocks_for(int64_t n) {
    int64_t b = (n + kBlock - 1) / kBlock;
    const int64_t cap = (int64_t)cu_count() * 32;
    return (unsigned)(b < 1 ? 1 : (b > cap ? cap : b));
}

int64_t nelem(const dt_tensor* t) { return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]; }

bool float_type(int32_t t) { return t == DT_TYPE_F32 || t == DT_TYPE_F16 || t == DT_TYPE_BF16; }

int check_desc(const dt_tensor* t, const char* who, const char* name, bool allow_i32 = false) {
    if (!t) return fail(DT_ERR_INVALID_ARG, "%s: %s is null", who, name);
    if (!float_type(t->type) && !(allow_i32 && t->type == DT_TYPE_I32))
        return fail(DT_ERR_UNSUPPORTED, "%s: %s has type %d (need F32/F16/BF16)", who, name, t->type);
    for (int i = 0; i < 4; ++i)
        if (t->ne[i] < 1) return fail(DT_ERR_INVALID_ARG, "%s: %s ne[%d] = %lld", who, name, i, (long long)t->ne[i]);
    if (!t->data) return fail(DT_ERR_INVALID_ARG, "%s: %s has no data", who, name);
    return DT_OK;
}

}  // namespace
}  // namespace dit

#define DT_CHECK_DESC(t, who, name)                          \
    do {                                                     \
        int rc_ = dit::check_desc((t), (who), (name));       \
        if (rc_) return rc_;                                 \
    } while (0)

// Same-type copies and concats move raw elements, so I32 is accepted there.
#define DT_CHECK_DESC_ANY(t, who, name)                      \
    do {                                                     \
        int rc_ = dit::check_desc((t), (who), (name), true); \
        if (rc_) return rc_;                                 \
    } while (0)

extern "C" int dt_op_binary(int32_t op, const dt_tensor* src0, const dt_tensor* src1,
                            const dt_tensor* dst, dt_stream_t stream) {
    DT_CHECK_DESC(src0, "dt_op_binary", "src0");
    DT_CHECK_DESC(src1, "dt_op_binary", "src1");
    DT_CHECK_DESC(dst, "dt_op_binary", "dst");
    DT_REQUIRE(op >= DT_BIN_ADD && op <= DT_BIN_DIV, "dt_op_binary: op %d", op);
    for (int i = 0; i < 4; ++i) {
        DT_REQUIRE(src0->ne[i] % src1->ne[i] == 0,
                   "dt_op_binary: src1 ne[%d]=%lld does not broadcast into src0 ne[%d]=%lld", i,
                   (long long)src1->ne[i], i, (long long)src0->ne[i]);
        DT_REQUIRE(dst->ne[i] == src0->ne[i], "dt_op_binary: dst shape differs from src0");
    }
    const int64_t n = dit::nelem(dst);
    hipLaunchKernelGGL(dit::binary_kernel, dim3(dit::blocks_for(n)), dim3(256), 0, (hipStream_t)stream,
                       op, dit::desc_of(src0), dit::desc_of(src1), dit::desc_of(dst), n);
    return dit::check_launch("dt_op_binary");
}

extern "C" int dt_op_unary(int32_t op, const dt_tensor* src, const dt_tensor* dst, float p0, float p1,
                           dt_stream_t stream) {
    DT_REQUIRE(op >= DT_UN_SIGMOID && op <= DT_UN_FILL, "dt_op_unary: op %d", op);
    DT_CHECK_DESC(dst, "dt_op_unary", "dst");
    dit::Desc a{};
    if (op != DT_UN_FILL) {
        DT_CHECK_DESC(src, "dt_op_unary", "src");
        DT_REQUIRE(dit::nelem(src) == dit::nelem(dst), "dt_op_unary: element counts differ");
        for (int i = 0; i < 4; ++i) DT_REQUIRE(src->ne[i] == dst->ne[i], "dt_op_unary: shapes differ");
        a = dit::desc_of(src);
    }
    const int64_t n = dit::nelem(dst);
    hipLaunchKernelGGL(dit::unary_kernel, dim3(dit::blocks_for(n)), dim3(256), 0, (hipStream_t)stream,
                       op, a, dit::desc_of(dst), p0, p1, n);
    return dit::check_launch("dt_op_unary");
}

static int norm_common(const dt_tensor* src, const dt_tensor* dst, float eps, int rms,
                       dt_stream_t stream, const char* who) {
    DT_CHECK_DESC(src, who, "src");
    DT_CHECK_DESC(dst, who, "dst");
    for (int i = 0; i < 4; ++i) DT_REQUIRE(src->ne[i] == dst->ne[i], "%s: shapes differ", who);
    const int64_t rows = src->ne[1] * src->ne[2] * src->ne[3];
    DT_REQUIRE(rows < (1ll << 31), "%s: too many rows", who);
    hipLaunchKernelGGL(dit::norm_kernel, dim3((unsigned)rows), dim3(256), 0, (hipStream_t)stream,
                       dit::desc_of(src), dit::desc_of(dst), eps, rms);
    return dit::check_launch(who);
}

extern "C" int dt_op_norm(const dt_tensor* src, const dt_tensor* dst, float eps, dt_stream_t stream) {
    return norm_common(src, dst, eps, 0, stream, "dt_op_norm");
}

extern "C" int dt_op_rms_norm(const dt_tensor* src, const dt_tensor* dst, float eps, dt_stream_t stream) {
    return norm_common(src, dst, eps, 1, stream, "dt_op_rms_norm");
}

extern "C" int dt_op_rope_ext(const dt_tensor* src, const int32_t* pos, const dt_tensor* dst,
                              int32_t n_dims, int32_t mode, float freq_base, float freq_scale,
                              float ext_factor, float attn_factor, dt_stream_t stream) {
    DT_CHECK_DESC(src, "dt_op_rope_ext", "src");
    DT_CHECK_DESC(dst, "dt_op_rope_ext", "dst");
    DT_REQUIRE(pos != nullptr, "dt_op_rope_ext: null pos");
    DT_REQUIRE(mode == 0, "dt_op_rope_ext: only mode 0 (NORMAL) is implemented, got %d", mode);
    DT_REQUIRE(ext_factor == 0.0f, "dt_op_rope_ext: ext_factor != 0 (YaRN) is not implemented");
    DT_REQUIRE(src->ne[0] % 2 == 0 && n_dims > 0 && n_dims % 2 == 0 && n_dims <= src->ne[0],
               "dt_op_rope_ext: bad n_dims %d for ne0 %lld", n_dims, (long long)src->ne[0]);
    for (int i = 0; i < 4; ++i) DT_REQUIRE(src->ne[i] == dst->ne[i], "dt_op_rope_ext: shapes differ");
    const int64_t n_pairs = dit::nelem(src) / 2;
    const float theta_scale = powf(freq_base, -2.0f / (float)n_dims);
    hipLaunchKernelGGL(dit::rope_kernel, dim3(dit::blocks_for(n_pairs)), dim3(256), 0,
                       (hipStream_t)stream, dit::desc_of(src), dit::desc_of(dst), pos, n_dims,
                       theta_scale, freq_scale, attn_factor, n_pairs);
    return dit::check_launch("dt_op_rope_ext");
}

extern "C" int dt_op_concat(const dt_tensor* a, const dt_tensor* b, int32_t dim, const dt_tensor* dst,
                            dt_stream_t stream) {
    DT_CHECK_DESC_ANY(a, "dt_op_concat", "a");
    DT_CHECK_DESC_ANY(b, "dt_op_concat", "b");
    DT_CHECK_DESC_ANY(dst, "dt_op_concat", "dst");
    const bool raw = a->type == b->type && a->type == dst->type;
    DT_REQUIRE(raw || (dit::float_type(a->type) && dit::float_type(b->type) && dit::float_type(dst->type)),
               "dt_op_concat: I32 operands must all be I32");
    DT_REQUIRE(dim >= 0 && dim < 4, "dt_op_concat: dim %d", dim);
    for (int i = 0; i < 4; ++i) {
        if (i == dim)
            DT_REQUIRE(dst->ne[i] == a->ne[i] + b->ne[i], "dt_op_concat: dst ne[%d] mismatch", i);
        else
            DT_REQUIRE(a->ne[i] == b->ne[i] && dst->ne[i] == a->ne[i], "dt_op_concat: ne[%d] mismatch", i);
    }
    const int64_t n = dit::nelem(dst);
    if (raw) {
        const int es = dit::elem_size(a->type);
        auto dense = [es](const dt_tensor* t) {
            int64_t want = es;
            for (int i = 0; i < 4; ++i) {
                if (t->ne[i] > 1 && t->nb[i] != want) return false;
                want *= t->ne[i];
            }
            return true;
        };
        int64_t ca = es, cb = es;  // bytes of one run of a / b: dims 0..dim
        for (int i = 0; i <= dim; ++i) {
            ca *= a->ne[i];
            cb *= b->ne[i];
        }
        if (n > 0 && dense(a) && dense(b) && dense(dst) && ca % 16 == 0 && cb % 16 == 0 && dit::aligned16(a->data) &&
            dit::aligned16(b->data) && dit::aligned16(dst->data)) {
            const int64_t nv = n * es / 16;
            hipLaunchKernelGGL(dit::concat_dense16_kernel, dim3(dit::blocks_for(nv)), dim3(256), 0,
                               (hipStream_t)stream, (const uint4*)a->data, (const uint4*)b->data, (uint4*)dst->data,
                               ca / 16, cb / 16, nv);
            return dit::check_launch("dt_op_concat");
        }
    }
    if (raw)
        hipLaunchKernelGGL(dit::concat_raw_kernel, dim3(dit::blocks_for(n)), dim3(256), 0,
                           (hipStream_t)stream, dit::desc_of(a), dit::desc_of(b), dit::desc_of(dst),
                           (int)dim, dit::elem_size(a->type), n);
    else
        hipLaunchKernelGGL(dit::concat_kernel, dim3(dit::blocks_for(n)), dim3(256), 0, (hipStream_t)stream,
                           dit::desc_of(a), dit::desc_of(b), dit::desc_of(dst), (int)dim, n);
    return dit::check_launch("dt_op_concat");
}

extern "C" int dt_op_cpy(const dt_tensor* src, const dt_tensor* dst, dt_stream_t stream) {
    DT_CHECK_DESC_ANY(src, "dt_op_cpy", "src");
    DT_CHECK_DESC_ANY(dst, "dt_op_cpy", "dst");
    DT_REQUIRE(dit::nelem(src) == dit::nelem(dst), "dt_op_cpy: element counts differ");
    const bool raw = src->type == dst->type;
    DT_REQUIRE(raw || (dit::float_type(src->type) && dit::float_type(dst->type)),
               "dt_op_cpy: I32 converts to I32 only");
    const int64_t n = dit::nelem(dst);
    if (raw)
        hipLaunchKernelGGL(dit::cpy_raw_kernel, dim3(dit::blocks_for(n)), dim3(256), 0,
                           (hipStream_t)stream, dit::desc_of(src), dit::desc_of(dst),
                           dit::elem_size(src->type), n);
    else
        hipLaunchKernelGGL(dit::cpy_kernel, dim3(dit::blocks_for(n)), dim3(256), 0, (hipStream_t)stream,
                           dit::desc_of(src), dit::desc_of(dst), n);
    return dit::check_launch("dt_op_cpy");
}
