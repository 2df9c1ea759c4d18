// hip_runtime.cpp -- HipRuntime: records dt_tensor nodes through the
// Runtime interface (src/ggml/Runtime.hpp) and executes them with the C ABI.
//
// compute() mirrors the reference's ExecutionRuntime::run
// (src/ggml/ExecutionRuntime.cpp:42-276) for one scope: leaves (inputs and
// parameters) get their own buffer and are uploaded, op nodes share one
// arena allocated with liveness reuse (ggml_gallocr's job in the reference,
// Context.hpp:118-135), nodes a fused kernel absorbs get no memory at all
// (dt_graph_plan tells which), and dt_graph_compute runs the graph.
#include "runtime.hpp"

#include <algorithm>
#include <cstring>
#include <limits>
#include <map>

namespace dit {
namespace host {

void check(int rc, const char* what) {
    if (rc != DT_OK) throw Error(std::string(what) + ": " + dt_last_error());
}

namespace {

thread_local Runtime* g_current = nullptr;

int32_t fbits(float f) {
    int32_t i;
    std::memcpy(&i, &f, 4);
    return i;
}

int64_t elem_size(int32_t type) {
    switch (type) {
        case DT_TYPE_F32:
        case DT_TYPE_I32:
            return 4;
        case DT_TYPE_F16:
        case DT_TYPE_BF16:
            return 2;
        case DT_TYPE_Q8_0_SPLIT:  // one code byte per element; scales follow the codes
            return 1;
        case DT_TYPE_CONV2D_PACKED:  // bf16 elements in dt_conv2d's padded tile order
            return 2;
        default:
            return 0;
    }
}

// Block size (elements) and bytes per block of the quantised types.
void block_layout(int32_t type, int64_t* qk, int64_t* bytes) {
    if (type == DT_TYPE_Q8_0) {
        *qk = 32;
        *bytes = 34;
    } else if (type == DT_TYPE_Q4_K) {
        *qk = 256;
        *bytes = 144;
    } else {
        *qk = 1;
        *bytes = elem_size(type);
    }
}

void contiguous_nb(int32_t type, const int64_t ne[4], int64_t nb[4]) {
    int64_t qk, bs;
    block_layout(type, &qk, &bs);
    nb[0] = bs;
    nb[1] = nb[0] * (ne[0] / qk);
    nb[2] = nb[1] * ne[1];
    nb[3] = nb[2] * ne[2];
}

bool is_contiguous(const Node* t) {
    int64_t nb[4];
    contiguous_nb(t->type, t->ne, nb);
    for (int i = 0; i < 4; ++i)
        if (t->ne[i] > 1 && t->nb[i] != nb[i]) return false;
    return true;
}

int64_t nelements(const Node* t) { return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]; }

constexpr size_t kAlign = 256;
size_t align_up(size_t n) { return (n + kAlign - 1) / kAlign * kAlign; }

// Best-fit free list over [0, peak) with coalescing.
class ArenaPlanner {
public:
    size_t alloc(size_t n) {
        n = align_up(n ? n : 1);
        auto best = free_.end();
        for (auto it = free_.begin(); it != free_.end(); ++it)
            if (it->second >= n && (best == free_.end() || it->second < best->second)) best = it;
        if (best != free_.end()) {
            const size_t off = best->first, sz = best->second;
            free_.erase(best);
            if (sz > n) free_[off + n] = sz - n;
            return off;
        }
        // Grow: reuse a free block that touches the end.
        size_t off = peak_;
        if (!free_.empty()) {
            auto last = std::prev(free_.end());
            if (last->first + last->second == peak_) {
                off = last->first;
                free_.erase(last);
            }
        }
        peak_ = off + n;
        return off;
    }
    void release(size_t off, size_t n) {
        n = align_up(n ? n : 1);
        auto it = free_.emplace(off, n).first;
        auto next = std::next(it);
        if (next != free_.end() && it->first + it->second == next->first) {
            it->second += next->second;
            free_.erase(next);
        }
        if (it != free_.begin()) {
            auto prev = std::prev(it);
            if (prev->first + prev->second == it->first) {
                prev->second += it->second;
                free_.erase(it);
            }
        }
    }
    size_t peak() const { return peak_; }

private:
    std::map<size_t, size_t> free_;
    size_t peak_ = 0;
};

}  // namespace

Runtime& current_runtime() {
    if (!g_current) throw std::logic_error("no Runtime in scope (create a RuntimeScope)");
    return *g_current;
}

RuntimeScope::RuntimeScope(Runtime& rt) : prev_(g_current) { g_current = &rt; }
RuntimeScope::~RuntimeScope() { g_current = prev_; }

// ---------------------------------------------------------------------------

HipRuntime::HipRuntime(int device, dt_stream_t stream) {
    if (device < 0) return;
    check(dt_backend_init(device, &be_), "dt_backend_init");
    check(dt_backend_set_stream(be_, stream), "dt_backend_set_stream");
}

HipRuntime::~HipRuntime() {
    try {
        reset();
    } catch (...) {
    }
    if (exec_) dt_graph_exec_free(exec_);
    if (be_) dt_backend_free(be_);
}

size_t HipRuntime::nbytes(const Node* t) {
    if (t->type == DT_TYPE_Q8_0_SPLIT) return (size_t)dt_q8_0_split_bytes(t->ne[1] * t->ne[2] * t->ne[3], t->ne[0]);
    if (t->type == DT_TYPE_CONV2D_PACKED) return dt_conv2d_packed_bytes(t->ne[3], t->ne[2], t->ne[0]);
    int64_t qk, bs;
    block_layout(t->type, &qk, &bs);
    return (size_t)(nelements(t) / qk * bs);
}

Node* HipRuntime::make(int32_t type, const int64_t ne[4], int32_t op) {
    nodes_.emplace_back();
    Node* t = &nodes_.back();
    std::memset(t, 0, sizeof(Node));
    t->type = type;
    t->op = op;
    for (int i = 0; i < 4; ++i) t->ne[i] = ne[i];
    contiguous_nb(type, t->ne, t->nb);
    t->id = (int32_t)nodes_.size() - 1;
    if (op != DT_OP_NONE) order_.push_back(t);
    prepared_ = false;
    return t;
}

Node* HipRuntime::view_of(Node* src, const int64_t ne[4], const int64_t nb[4], size_t offset) {
    Node* t = make(src->type, ne, DT_OP_VIEW);
    for (int i = 0; i < 4; ++i) t->nb[i] = nb[i];
    t->src[0] = src;
    t->op_params[0] = (int32_t)(uint32_t)(offset & 0xFFFFFFFFu);
    t->op_params[1] = (int32_t)(offset >> 32);
    return t;
}

Node* HipRuntime::root_of(Node* t) const {
    for (;;) {
        if (t->op == DT_OP_VIEW) {
            t = t->src[0];
            continue;
        }
        auto a = alias_.find(t);
        if (a != alias_.end()) {
            t = a->second;
            continue;
        }
        return t;
    }
}

// ---- creation ----------------------------------------------------------------

Node* HipRuntime::new_tensor(int32_t type, int n_dims, const int64_t* ne) {
    if (n_dims < 1 || n_dims > 4) throw std::invalid_argument("new_tensor: n_dims must be 1..4");
    int64_t e[4] = {1, 1, 1, 1};
    for (int i = 0; i < n_dims; ++i) e[i] = ne[i];
    Node* t = make(type, e, DT_OP_NONE);
    leaves_.push_back(t);
    return t;
}

Node* HipRuntime::new_tensor_1d(int32_t type, int64_t ne0) { return new_tensor(type, 1, &ne0); }

void HipRuntime::set_input(Node* t) { (void)t; }
void HipRuntime::set_param(Node* t) { (void)t; }
void HipRuntime::set_output(Node* t) { t->flags |= DT_FLAG_OUTPUT; }

Node* HipRuntime::fill(Node* t, float value) {
    Node* r = make(t->type, t->ne, DT_OP_FILL);
    r->op_params[0] = fbits(value);
    return r;
}

// ---- copies ------------------------------------------------------------------

Node* HipRuntime::cont(Node* t) {
    Node* r = make(t->type, t->ne, DT_OP_CPY);
    r->src[0] = t;
    return r;
}

Node* HipRuntime::dup(Node* t) { return cont(t); }

Node* HipRuntime::cast(Node* t, int32_t type) {
    Node* r = make(type, t->ne, DT_OP_CPY);
    r->src[0] = t;
    return r;
}

Node* HipRuntime::cpy(Node* src, Node* dst) {
    if (nelements(src) != nelements(dst)) throw std::invalid_argument("cpy: element counts differ");
    Node* r = make(dst->type, dst->ne, DT_OP_CPY);
    for (int i = 0; i < 4; ++i) r->nb[i] = dst->nb[i];
    r->src[0] = src;
    r->src[1] = dst;
    alias_[r] = dst;
    return r;
}

// ---- elementwise ---------------------------------------------------------------

Node* HipRuntime::unary(Node* a, int32_t kind, float p0, float p1) {
    Node* r = make(a->type, a->ne, DT_OP_UNARY);
    r->src[0] = a;
    r->op_params[0] = kind;
    r->op_params[1] = fbits(p0);
    r->op_params[2] = fbits(p1);
    return r;
}

Node* HipRuntime::sqrt(Node* t) { return unary(t, DT_UN_SQRT); }
Node* HipRuntime::exp(Node* t) { return unary(t, DT_UN_EXP); }
Node* HipRuntime::log(Node* t) { return unary(t, DT_UN_LOG); }
Node* HipRuntime::sin(Node* t) { return unary(t, DT_UN_SIN); }
Node* HipRuntime::cos(Node* t) { return unary(t, DT_UN_COS); }

Node* HipRuntime::sigmoid(Node* t) {
    Node* r = make(t->type, t->ne, DT_OP_SIGMOID);
    r->src[0] = t;
    return r;
}

Node* HipRuntime::binary(int32_t op, Node* a, Node* b) {
    for (int i = 0; i < 4; ++i)
        if (b->ne[i] == 0 || a->ne[i] % b->ne[i] != 0)
            throw std::invalid_argument("binary op: rhs does not broadcast into lhs");
    Node* r = make(a->type, a->ne, op);
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

Node* HipRuntime::add(Node* a, Node* b) { return binary(DT_OP_ADD, a, b); }
Node* HipRuntime::sub(Node* a, Node* b) { return binary(DT_OP_SUB, a, b); }
Node* HipRuntime::mul(Node* a, Node* b) { return binary(DT_OP_MUL, a, b); }
Node* HipRuntime::div(Node* a, Node* b) { return binary(DT_OP_DIV, a, b); }

Node* HipRuntime::scale(Node* t, float value) {
    Node* r = make(t->type, t->ne, DT_OP_SCALE);
    r->src[0] = t;
    r->op_params[0] = fbits(value);
    return r;
}

Node* HipRuntime::clamp(Node* t, float mn, float mx) { return unary(t, DT_UN_CLAMP, mn, mx); }

// ggml_mul_mat(w, x) (Runtime.hpp:136-139; Linear.cpp:24): y = x W^T over
// ne0.  F32 weights with F32 activations (the reference's precision) stay
// F32: the fp32 GEMM.  Otherwise the bf16 MFMA GEMM takes BF16 activations
// and BF16 or Q8_0_SPLIT weights (Q8_0 dequantised to bf16 inside the GEMM):
// an F32 activation is cast to BF16 by a CPY node first (ggml's CPU backend
// likewise converts the activation to the weight's vec_dot type), and the
// result is F32 when the activation was F32 (ggml's result type) or BF16 for
// BF16 activations.
Node* HipRuntime::mul_mat(Node* w, Node* x) {
    if (w->ne[0] != x->ne[0]) throw std::invalid_argument("mul_mat: ne0 (K) of weight and input differ");
    if (w->ne[2] != 1 || w->ne[3] != 1) throw Unsupported("mul_mat: batched weights are not supported");
    if (w->type == DT_TYPE_Q8_0 || w->type == DT_TYPE_Q4_K)
        throw Unsupported("mul_mat: repack Q8_0 weights once at load (dt_q8_0_split -> DT_TYPE_Q8_0_SPLIT) or "
                          "dequantise them to BF16 (dt_dequant)");
    const int32_t out_type = x->type == DT_TYPE_BF16 ? DT_TYPE_BF16 : DT_TYPE_F32;
    if (w->type == DT_TYPE_F32 && x->type == DT_TYPE_F32) {
        if (w->nb[0] != 4) w = cont(w);
        if (x->nb[0] != 4) x = cont(x);
    } else {
        if (w->type != DT_TYPE_BF16 && w->type != DT_TYPE_Q8_0_SPLIT) w = cast(w, DT_TYPE_BF16);
        if (x->type != DT_TYPE_BF16) x = cast(x, DT_TYPE_BF16);
        else if (x->nb[0] != 2) x = cont(x);
    }
    const int64_t ne[4] = {w->ne[1], x->ne[1], x->ne[2], x->ne[3]};
    Node* r = make(out_type, ne, DT_OP_MUL_MAT);
    r->src[0] = w;
    r->src[1] = x;
    return r;
}

// ---- views -----------------------------------------------------------------------

static void reshape_check(const Node* t, const int64_t ne[4]) {
    if (!is_contiguous(t)) throw std::invalid_argument("reshape: tensor is not contiguous");
    if (ne[0] * ne[1] * ne[2] * ne[3] != nelements(t))
        throw std::invalid_argument("reshape: element count changes");
}

Node* HipRuntime::reshape_4d(Node* t, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3) {
    const int64_t ne[4] = {ne0, ne1, ne2, ne3};
    reshape_check(t, ne);
    int64_t nb[4];
    contiguous_nb(t->type, ne, nb);
    return view_of(t, ne, nb, 0);
}
Node* HipRuntime::reshape_1d(Node* t, int64_t ne0) { return reshape_4d(t, ne0, 1, 1, 1); }
Node* HipRuntime::reshape_2d(Node* t, int64_t ne0, int64_t ne1) { return reshape_4d(t, ne0, ne1, 1, 1); }
Node* HipRuntime::reshape_3d(Node* t, int64_t ne0, int64_t ne1, int64_t ne2) {
    return reshape_4d(t, ne0, ne1, ne2, 1);
}

Node* HipRuntime::permute(Node* t, int a0, int a1, int a2, int a3) {
    const int ax[4] = {a0, a1, a2, a3};
    int64_t ne[4], nb[4];
    bool seen[4] = {false, false, false, false};
    for (int i = 0; i < 4; ++i) {
        if (ax[i] < 0 || ax[i] > 3 || seen[ax[i]]) throw std::invalid_argument("permute: bad axes");
        seen[ax[i]] = true;
        ne[ax[i]] = t->ne[i];
        nb[ax[i]] = t->nb[i];
    }
    return view_of(t, ne, nb, 0);
}

Node* HipRuntime::view_4d(Node* t, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3, size_t nb1,
                          size_t nb2, size_t nb3, size_t offset) {
    const int64_t ne[4] = {ne0, ne1, ne2, ne3};
    const int64_t nb[4] = {t->nb[0], (int64_t)nb1, (int64_t)nb2, (int64_t)nb3};
    return view_of(t, ne, nb, offset);
}
Node* HipRuntime::view_3d(Node* t, int64_t ne0, int64_t ne1, int64_t ne2, size_t nb1, size_t nb2,
                          size_t offset) {
    return view_4d(t, ne0, ne1, ne2, 1, nb1, nb2, nb2 * ne2, offset);
}
Node* HipRuntime::view_2d(Node* t, int64_t ne0, int64_t ne1, size_t nb1, size_t offset) {
    return view_4d(t, ne0, ne1, 1, 1, nb1, nb1 * ne1, nb1 * ne1, offset);
}
Node* HipRuntime::view_1d(Node* t, int64_t ne0, size_t offset) {
    const size_t row = (size_t)(t->nb[0] * ne0);
    return view_4d(t, ne0, 1, 1, 1, row, row, row, offset);
}

// ---- structure ---------------------------------------------------------------------

Node* HipRuntime::repeat(Node* t, Node* target) {
    // ggml_repeat tiles t into target's shape: a broadcast add onto zeros.
    Node* zeros = make(t->type, target->ne, DT_OP_FILL);
    zeros->op_params[0] = fbits(0.0f);
    return binary(DT_OP_ADD, zeros, t);
}

Node* HipRuntime::concat(Node* a, Node* b, int dim) {
    if (dim < 0 || dim > 3) throw std::invalid_argument("concat: dim must be 0..3");
    int64_t ne[4];
    for (int i = 0; i < 4; ++i) {
        if (i != dim && a->ne[i] != b->ne[i]) throw std::invalid_argument("concat: shapes differ");
        ne[i] = a->ne[i] + (i == dim ? b->ne[i] : 0);
    }
    Node* r = make(a->type, ne, DT_OP_CONCAT);
    r->src[0] = a;
    r->src[1] = b;
    r->op_params[0] = dim;
    return r;
}

Node* HipRuntime::sum_rows(Node*) { throw Unsupported("sum_rows: not part of the DiT elementwise chain"); }
// ggml_flash_attn_ext (Runtime.hpp:250-257; FlashAttentionOp.cpp:84-94):
// q ne {D, Sq, H, B}, k / v ne {D, Skv, H, B} -> ne {D, H, Sq, B}.  No mask,
// ALiBi or softcap (Flux2 uses none).  F32 q, k and v stay F32 (the fp32
// attention, F32 result); otherwise F32 operands are cast to BF16 and give
// an F32 result, BF16 operands a BF16 result.
Node* HipRuntime::flash_attn_ext(Node* q, Node* k, Node* v, Node* mask, float scale, float max_bias,
                                 float logit_softcap) {
    if (mask) throw Unsupported("flash_attn_ext: masks are not supported");
    if (max_bias != 0.0f || logit_softcap != 0.0f)
        throw Unsupported("flash_attn_ext: ALiBi / logit softcap are not supported");
    if (q->ne[0] != 128 || k->ne[0] != 128 || v->ne[0] != 128)
        throw Unsupported("flash_attn_ext: head_dim 128 only");
    const int32_t out_type = q->type == DT_TYPE_BF16 ? DT_TYPE_BF16 : DT_TYPE_F32;
    const bool f32 = q->type == DT_TYPE_F32 && k->type == DT_TYPE_F32 && v->type == DT_TYPE_F32;
    auto prep = [&](Node* t) {
        if (f32) return t->nb[0] != 4 ? cont(t) : t;
        return t->type != DT_TYPE_BF16 ? cast(t, DT_TYPE_BF16) : t->nb[0] != 2 ? cont(t) : t;
    };
    q = prep(q);
    k = prep(k);
    v = prep(v);
    const int64_t ne[4] = {q->ne[0], q->ne[2], q->ne[1], q->ne[3]};
    Node* r = make(out_type, ne, DT_OP_FLASH_ATTN_EXT);
    r->src[0] = q;
    r->src[1] = k;
    r->src[2] = v;
    r->op_params[0] = fbits(scale);
    return r;
}
// ggml_conv_2d_direct (Runtime.hpp, Conv2d.cpp:38-52): weight a ne {K, K, Ci, Co},
// contiguous input b ne {W, H, Ci, N} -> ne {W', H', Co, N} of b's type.  The
// VAE decoder's convolutions only: stride 1, dilation 1, K in {1, 3} with
// "same" padding (K - 1) / 2.
Node* HipRuntime::conv_2d_direct(Node* a, Node* b, int s0, int s1, int p0, int p1, int d0, int d1) {
    const int64_t K = a->ne[0];
    if (s0 != 1 || s1 != 1 || d0 != 1 || d1 != 1)
        throw Unsupported("conv_2d_direct: stride and dilation 1 only");
    if (a->ne[1] != K || (K != 1 && K != 3) || p0 != (K - 1) / 2 || p1 != (K - 1) / 2)
        throw Unsupported("conv_2d_direct: square 1x1 / 3x3 kernels with padding (K - 1) / 2 only");
    if (a->ne[2] != b->ne[2]) throw std::invalid_argument("conv_2d_direct: weight and input channels differ");
    if (a->type != DT_TYPE_F32 && a->type != DT_TYPE_BF16 && a->type != DT_TYPE_CONV2D_PACKED)
        throw Unsupported("conv_2d_direct: F32 / BF16 or packed weights only");
    if (b->type != DT_TYPE_F32 && b->type != DT_TYPE_BF16)
        throw Unsupported("conv_2d_direct: F32 / BF16 input only");
    if (a->type == DT_TYPE_CONV2D_PACKED && (a->op != DT_OP_NONE || !is_contiguous(a)))
        throw std::invalid_argument("conv_2d_direct: a packed weight must be the whole leaf");
    if (!is_contiguous(a)) a = cont(a);
    if (!is_contiguous(b)) b = cont(b);
    const int64_t ne[4] = {b->ne[0], b->ne[1], a->ne[3], b->ne[3]};
    Node* r = make(b->type, ne, DT_OP_CONV_2D_DIRECT);
    r->src[0] = a;
    r->src[1] = b;
    const int32_t params[6] = {s0, s1, p0, p1, d0, d1};
    for (int i = 0; i < 6; ++i) r->op_params[i] = params[i];
    return r;
}
Node* HipRuntime::get_rows(Node*, Node*) { throw Unsupported("get_rows: not part of the DiT elementwise chain"); }
Node* HipRuntime::pool_2d(Node*, PoolOp, int, int, int, int, float, float) {
    throw Unsupported("pool_2d: not part of the DiT elementwise chain");
}
Node* HipRuntime::interpolate(Node*, int64_t, int64_t, int64_t, int64_t, uint32_t) {
    throw Unsupported("interpolate: not part of the DiT elementwise chain");
}
// ggml_upscale(a, factor, NEAREST) (Upsample2D.cpp:36-63): ne {W, H, C, N}
// -> {factor W, factor H, C, N}, each output pixel its source pixel's value.
Node* HipRuntime::upscale(Node* a, int scale_factor, ScaleMode mode) {
    if (mode != ScaleMode::Nearest) throw Unsupported("upscale: nearest mode only");
    if (scale_factor < 1) throw std::invalid_argument("upscale: factor must be >= 1");
    if (!is_contiguous(a)) a = cont(a);
    const int64_t ne[4] = {a->ne[0] * scale_factor, a->ne[1] * scale_factor, a->ne[2], a->ne[3]};
    Node* r = make(a->type, ne, DT_OP_UPSCALE);
    r->src[0] = a;
    r->op_params[0] = scale_factor;
    return r;
}

// ---- norms / rope ----------------------------------------------------------------

Node* HipRuntime::norm(Node* a, float eps) {
    Node* r = make(a->type, a->ne, DT_OP_NORM);
    r->src[0] = a;
    r->op_params[0] = fbits(eps);
    return r;
}

Node* HipRuntime::rms_norm(Node* a, float eps) {
    Node* r = make(a->type, a->ne, DT_OP_RMS_NORM);
    r->src[0] = a;
    r->op_params[0] = fbits(eps);
    return r;
}

Node* HipRuntime::rope_ext(Node* a, Node* b, Node* c, int n_dims, int mode, int n_ctx_orig,
                           float freq_base, float freq_scale, float ext_factor, float attn_factor,
                           float beta_fast, float beta_slow) {
    (void)n_ctx_orig;
    (void)beta_fast;
    (void)beta_slow;
    if (c != nullptr) throw Unsupported("rope_ext: frequency factors are not supported");
    if (mode != 0) throw Unsupported("rope_ext: only mode 0 (NORMAL) is supported");
    if (ext_factor != 0.0f) throw Unsupported("rope_ext: YaRN (ext_factor != 0) is not supported");
    if (!b || b->type != DT_TYPE_I32 || b->ne[0] != a->ne[2])
        throw std::invalid_argument("rope_ext: positions must be I32 with ne0 == a->ne[2]");
    Node* r = make(a->type, a->ne, DT_OP_ROPE);
    r->src[0] = a;
    r->src[1] = b;
    r->op_params[0] = n_dims;
    r->op_params[1] = mode;
    r->op_params[2] = fbits(freq_base);
    r->op_params[3] = fbits(freq_scale);
    r->op_params[4] = fbits(ext_factor);
    r->op_params[5] = fbits(attn_factor);
    return r;
}

// ---- data and execution ----------------------------------------------------------

void HipRuntime::bind(Node* leaf, const void* host, size_t bytes) {
    if (leaf->op != DT_OP_NONE) throw std::invalid_argument("bind: only leaves carry host data");
    if (bytes != nbytes(leaf)) throw std::invalid_argument("bind: byte count does not match the tensor");
    auto& v = host_data_[leaf];
    v.assign((const uint8_t*)host, (const uint8_t*)host + bytes);
    if (device_data_.erase(leaf)) prepared_ = false;
}

void HipRuntime::bind_device(Node* leaf, void* device_ptr) {
    if (leaf->op != DT_OP_NONE) throw std::invalid_argument("bind_device: only leaves carry data");
    if (!device_ptr) throw std::invalid_argument("bind_device: null pointer");
    host_data_.erase(leaf);
    device_data_[leaf] = device_ptr;
    leaf->data = device_ptr;
    prepared_ = false;
}

const ComputeStats& HipRuntime::plan() {
    prepare(false);
    return stats_;
}

void HipRuntime::upload_leaves() {
    for (Node* l : leaves_) {
        auto h = host_data_.find(l);
        if (h != host_data_.end())
            check(dt_tensor_set(l, h->second.data(), 0, h->second.size(), nullptr), "dt_tensor_set");
    }
}

void HipRuntime::compute_graph() {
    if (!be_) throw Error("compute_graph: this runtime has no device");
    if (!prepared_ || !exec_ || exec_gen_ != plan_gen_) {
        compute();  // plans, allocates and creates the backend's scratch before the recording
        if (exec_) check(dt_graph_exec_free(exec_), "dt_graph_exec_free");
        exec_ = nullptr;
        const int n = (int)order_.size();
        if (n) check(dt_graph_capture_ex(be_, order_.data(), n, compute_flags(), &exec_), "dt_graph_capture");
        exec_gen_ = plan_gen_;
        return;
    }
    upload_leaves();
    check(dt_graph_exec_launch(be_, exec_), "dt_graph_exec_launch");
    check(dt_backend_synchronize(be_), "dt_backend_synchronize");
}

void HipRuntime::compute() {
    if (!be_) throw Error("compute: this runtime has no device");
    if (!prepared_) prepare();
    upload_leaves();
    const int n = (int)order_.size();
    if (n) check(dt_graph_compute_ex(be_, order_.data(), n, compute_flags()), "dt_graph_compute");
    check(dt_backend_synchronize(be_), "dt_backend_synchronize");
    int32_t k = 0, f = 0, held = 0;
    dt_graph_last_stats_ex(&k, &f, &held);
    stats_.kernels = k;
    stats_.fused_nodes = f;
    stats_.launches_held = held;
}

void HipRuntime::set_allocation(Allocation a) {
    if (a != alloc_) prepared_ = false;
    alloc_ = a;
}

namespace {
// Ops whose kernels may write their output over src[0] element for element
// (ggml-alloc's in-place candidates among the ops recorded here).
bool inplace_op(const Node* t) {
    switch (t->op) {
        case DT_OP_ADD:
        case DT_OP_SUB:
        case DT_OP_MUL:
        case DT_OP_DIV:
        case DT_OP_SCALE:
        case DT_OP_SIGMOID:
        case DT_OP_UNARY:
        case DT_OP_NORM:
        case DT_OP_RMS_NORM:
            return true;
        default:
            return false;
    }
}
}  // namespace

void HipRuntime::prepare(bool allocate) {
    ++plan_gen_;
    const int n = (int)order_.size();
    // 1. fusion plan: which nodes are absorbed (no storage) and where every
    //    node's kernel runs (absorbed -> its root, grouped GEMMs -> the
    //    group's first member)
    std::vector<int32_t> fused_into(n, -1), runs_at(n, 0);
    if (n) check(dt_graph_plan_ex(order_.data(), n, fused_into.data(), runs_at.data()), "dt_graph_plan_ex");
    const bool node_order = alloc_ == Allocation::NodeOrder;
    std::vector<int32_t> plan_fused = fused_into, plan_runs = runs_at;
    if (node_order)  // memory follows node order; the executor adapts its plan to it
        for (int i = 0; i < n; ++i) {
            fused_into[i] = -1;
            runs_at[i] = i;
        }

    // 2. last use of every storage root, at the position where the reading
    //    kernel runs
    const int kForever = std::numeric_limits<int>::max();
    std::unordered_map<const Node*, int> last_use;
    for (int i = 0; i < n; ++i) {
        Node* t = order_[i];
        const int at = runs_at[i];
        for (int s = 0; s < 4; ++s) {
            if (!t->src[s]) continue;
            const Node* r = root_of(t->src[s]);
            int& lu = last_use[r];
            lu = std::max(lu, at);
        }
        if (t->flags & DT_FLAG_OUTPUT) last_use[root_of(t)] = kForever;
    }

    // 3. arena plan for op nodes that own storage: each output is placed at
    //    the position its kernel runs (never later than the node itself)
    //    before that position's inputs are released, so a kernel never
    //    writes over what it reads.
    ArenaPlanner planner;
    std::unordered_map<const Node*, size_t> offset;
    std::vector<std::vector<const Node*>> alloc_at(n), release_at(n);
    size_t naive = 0;
    for (int i = 0; i < n; ++i) {
        Node* t = order_[i];
        const bool owns = t->op != DT_OP_VIEW && !alias_.count(t);
        if (owns) naive += align_up(nbytes(t));
        if (owns && fused_into[i] < 0) alloc_at[std::min(i, (int)runs_at[i])].push_back(t);
    }
    for (int p = 0; p < n; ++p) {
        for (const Node* t : alloc_at[p]) {
            // NodeOrder: over src[0]'s memory when t is its last reader and
            // the op can run in place (same size, not an output).
            const Node* s0 = t->src[0] ? root_of(const_cast<Node*>(t->src[0])) : nullptr;
            if (node_order && s0 && inplace_op(t) && s0 == t->src[0] && offset.count(s0) &&
                nbytes(s0) == nbytes(t) && last_use.count(s0) && last_use.at(s0) == p &&
                !(s0->flags & DT_FLAG_OUTPUT)) {
                offset[t] = offset.at(s0);
                auto& rel = release_at[p];
                rel.erase(std::remove(rel.begin(), rel.end(), s0), rel.end());
                auto lu = last_use.find(t);
                const int end = lu == last_use.end() ? p : lu->second;
                if (end != kForever) release_at[std::max(end, p)].push_back(t);
                continue;
            }
            offset[t] = planner.alloc(nbytes(t));
            auto lu = last_use.find(t);
            const int end = lu == last_use.end() ? p : lu->second;
            if (end != kForever) release_at[std::max(end, p)].push_back(t);
        }
        for (const Node* r : release_at[p]) planner.release(offset.at(r), nbytes(r));
        release_at[p].clear();
    }

    stats_.nodes = n;
    stats_.arena_bytes = planner.peak();
    stats_.naive_bytes = naive;
    stats_.fused_nodes = 0;
    stats_.mul_mat_nodes = stats_.attention_nodes = stats_.grouped_nodes = stats_.deferred_nodes = 0;
    for (int i = 0; i < n; ++i) {
        stats_.fused_nodes += plan_fused[i] >= 0;
        stats_.grouped_nodes += plan_fused[i] < 0 && plan_runs[i] < i;
        stats_.deferred_nodes += plan_fused[i] < 0 && plan_runs[i] > i;
        stats_.mul_mat_nodes += order_[i]->op == DT_OP_MUL_MAT;
        stats_.attention_nodes += order_[i]->op == DT_OP_FLASH_ATTN_EXT;
    }
    stats_.launches_held = 0;
    if (!allocate) {
        if (node_order && n) {
            // The executor's plan for this placement, on stand-in addresses
            // (leaves apart from the arena), without a device.  Every node's
            // and leaf's data pointer is restored afterwards, so a plan()
            // between two computes leaves the prepared placement in force.
            std::vector<void*> saved_leaves, saved_nodes;
            saved_leaves.reserve(leaves_.size());
            saved_nodes.reserve(order_.size());
            for (Node* l : leaves_) saved_leaves.push_back(l->data);
            for (Node* t : order_) saved_nodes.push_back(t->data);
            const uintptr_t kLeafBase = (uintptr_t)1 << 44, kArenaBase = (uintptr_t)1 << 40;
            size_t off = 0;
            for (Node* l : leaves_) {
                l->data = (void*)(kLeafBase + off);
                off += align_up(nbytes(l));
            }
            for (int i = 0; i < n; ++i) {
                auto o = offset.find(order_[i]);
                order_[i]->data = o != offset.end() ? (void*)(kArenaBase + o->second) : nullptr;
            }
            resolve_alias_data();
            std::vector<int32_t> cf(n), cr(n);
            int32_t held = 0;
            check(dt_graph_plan_checked(order_.data(), n, cf.data(), cr.data(), &held), "dt_graph_plan_checked");
            stats_.launches_held = held;
            stats_.fused_nodes_checked = 0;
            for (int i = 0; i < n; ++i) stats_.fused_nodes_checked += cf[i] >= 0;
            for (size_t i = 0; i < leaves_.size(); ++i) leaves_[i]->data = saved_leaves[i];
            for (size_t i = 0; i < order_.size(); ++i) order_[i]->data = saved_nodes[i];
        }
        return;
    }

    // 4. device memory: leaves in their own buffer, op nodes in the arena
    if (leaf_buf_) {
        check(dt_buffer_free(be_, leaf_buf_), "dt_buffer_free");
        leaf_buf_ = nullptr;
    }
    size_t leaf_bytes = 0;
    for (Node* l : leaves_)
        if (!device_data_.count(l)) leaf_bytes += align_up(nbytes(l));
    if (leaf_bytes) check(dt_buffer_alloc(be_, leaf_bytes, &leaf_buf_), "dt_buffer_alloc(leaves)");
    size_t off = 0;
    for (Node* l : leaves_) {
        auto d = device_data_.find(l);
        if (d != device_data_.end()) {
            l->data = d->second;
            continue;
        }
        l->data = (char*)leaf_buf_ + off;
        off += align_up(nbytes(l));
    }
    if (planner.peak() > arena_cap_) {
        if (arena_) check(dt_buffer_free(be_, arena_), "dt_buffer_free");
        arena_ = nullptr;
        arena_cap_ = 0;
        check(dt_buffer_alloc(be_, planner.peak(), &arena_), "dt_buffer_alloc(arena)");
        arena_cap_ = planner.peak();
    }
    for (int i = 0; i < n; ++i) {
        Node* t = order_[i];
        auto o = offset.find(t);
        t->data = o != offset.end() ? (char*)arena_ + o->second : nullptr;
    }
    resolve_alias_data();
    prepared_ = true;
}

// A CPY into a destination writes the destination's memory (a view's
// address resolved through its chain).
void HipRuntime::resolve_alias_data() {
    for (Node* t : order_) {
        if (!alias_.count(t)) continue;
        Node* r = t->src[1];
        int64_t extra = 0;
        while (r->op == DT_OP_VIEW) {
            extra += (int64_t)(uint32_t)r->op_params[0] | ((int64_t)r->op_params[1] << 32);
            r = r->src[0];
        }
        t->data = r->data ? (char*)r->data + extra : nullptr;
    }
}

void HipRuntime::read(const Node* node, void* host, size_t bytes) const {
    if (!node->data) throw std::invalid_argument("read: node has no data (was it marked as output?)");
    check(dt_tensor_get(node, host, 0, bytes, nullptr), "dt_tensor_get");
}

void HipRuntime::reset() {
    if (exec_) dt_graph_exec_free(exec_);
    exec_ = nullptr;
    if (be_ && leaf_buf_) dt_buffer_free(be_, leaf_buf_);
    if (be_ && arena_) dt_buffer_free(be_, arena_);
    leaf_buf_ = arena_ = nullptr;
    arena_cap_ = 0;
    nodes_.clear();
    order_.clear();
    leaves_.clear();
    host_data_.clear();
    device_data_.clear();
    prepared_ = false;
    alias_.clear();
    stats_ = ComputeStats();
}

}  // namespace host
}  // namespace dit
