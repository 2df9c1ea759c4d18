// graph.cpp -- dt_graph_compute: executes a ggml-shaped node list (the role
// of ggml_backend_graph_compute at src/ggml/ExecutionRuntime.cpp:227, 254)
// after a fusion pass that recognises the node chains the reference's
// modules emit and lowers each to one fused kernel:
//
//   adaLN           ADD(MUL(NORM(x), t[c]), shift[c])
//                   LayerNorm.cpp:17 + Flux2SingleTransformerBlock.hpp:53
//   gated residual  ADD(h, MUL(o, gate[c]))          Flux2SingleTransformerBlock.hpp:58
//   residual+adaLN  the adaLN chain whose x is a gated residual r: block i's
//                   residual feeding block i+1's norm, one pass writing r and
//                   the normalised output (r runs at the adaLN's position)
//   SwiGLU          MUL(MUL(g, SIGMOID(g)), u)        Flux2SwiGLU.hpp:20, SiLU.hpp:12
//   GroupNorm+SiLU  MUL(a, SIGMOID(a)), a = ADD(MUL(VIEW(NORM(VIEW(x))), w), b)
//                   GroupNorm.cpp:44-103 + SiLU.hpp:12 (affine / SiLU optional)
//   QK-RMSNorm+RoPE CONCAT*(ROPE(VIEW_a(MUL(RMS_NORM(q), w))), ...) along ne0
//                   RMSNorm.cpp:13-20 + Flux2PosEmbed.hpp:29-108, optionally
//                   with the txt|img CONCAT of Flux2Attention.hpp:114-116
//                   between the norm and the views.
//   GEMM accumulate ADD(y, MUL_MAT(w, x)): the second projection of
//                   Flux2FusedAttentionOutput.hpp:31-36 accumulates onto the
//                   first in the GEMM epilogue (dt_gemm_bf16 with addend).
//   Conv2d          ADD(CONV_2D_DIRECT(w, x), VIEW(bias)) with x optionally
//                   UPSCALE(x0, 2): Conv2d.cpp:38-102 and Upsample2D.cpp:50-72
//                   as one dt_conv2d (bias in the epilogue, the nearest
//                   upsample in the input addressing).
//
// After fusion, runs of independent MUL_MATs (only VIEWs between them, every
// input computed before the first) become one grouped GEMM launch at the
// first one's position: the q/k/v/gate/up projections Linear::forward issues
// back to back.  Those MUL_MATs keep their own outputs; dt_graph_plan_ex
// reports where each node's kernel runs so the caller keeps inputs alive and
// places outputs accordingly.
//
// MUL_MAT and FLASH_ATTN_EXT (Linear.cpp:24, FlashAttentionOp.cpp:84-94) run
// the bf16 MFMA kernels of gemm.hip and attention.hip.  An attention whose q
// is a QK-RMSNorm+RoPE chain used nowhere else takes that chain as its
// prologue (dt_flash_attn_qk_bf16: q is normalised and rotated as it is
// loaded, never stored); the block's k chain then joins its SwiGLU in one
// launch.
//
// A chain is fused only when every interior node is consumed solely inside
// the chain and is not flagged DT_FLAG_OUTPUT; everything else runs the
// unfused per-op kernels of ops.hip.
#include <algorithm>
#include <cstring>
#include <iterator>
#include <functional>
#include <map>
#include <unordered_map>
#include <vector>

#include "capi_util.hpp"
#include "dit_hip.h"
#include "kernels.hpp"

namespace dit {
namespace {

thread_local int g_kernels = 0;
thread_local int g_fused = 0;

float fparam(const dt_tensor* t, int i) {
    float f;
    std::memcpy(&f, &t->op_params[i], 4);
    return f;
}

// Byte offset of a VIEW into its source: op_params[0] (low) | op_params[1] (high).
int64_t view_offset(const dt_tensor* t) {
    return (int64_t)(uint32_t)t->op_params[0] | ((int64_t)t->op_params[1] << 32);
}

// Rows of ne[0] elements at a uniform row stride (in elements) covering
// dims 1..3.
bool row_layout(const dt_tensor* t, int64_t* rows, int64_t* stride) {
    const int es = elem_size(t->type);
    if (!es || t->nb[0] != es) return false;
    int64_t rs;
    if (t->ne[1] > 1) rs = t->nb[1];
    else if (t->ne[2] > 1) rs = t->nb[2];
    else if (t->ne[3] > 1) rs = t->nb[3];
    else rs = t->ne[0] * es;
    if (t->ne[1] > 1 && t->nb[1] != rs) return false;
    if (t->ne[2] > 1 && t->nb[2] != rs * t->ne[1]) return false;
    if (t->ne[3] > 1 && t->nb[3] != rs * t->ne[1] * t->ne[2]) return false;
    if (rs % es) return false;
    *rows = t->ne[1] * t->ne[2] * t->ne[3];
    *stride = rs / es;
    return true;
}

bool same_shape(const dt_tensor* a, const dt_tensor* b) {
    for (int i = 0; i < 4; ++i)
        if (a->ne[i] != b->ne[i]) return false;
    return true;
}

bool contiguous_f32(const dt_tensor* t) {
    return t->type == DT_TYPE_F32 && t->nb[0] == 4 &&
           (t->ne[1] == 1 || t->nb[1] == 4 * t->ne[0]) &&
           (t->ne[2] == 1 || t->nb[2] == 4 * t->ne[0] * t->ne[1]) &&
           (t->ne[3] == 1 || t->nb[3] == 4 * t->ne[0] * t->ne[1] * t->ne[2]);
}

// Every element in order, no gaps (any element type).
bool dense(const dt_tensor* t) {
    int64_t rows, stride;
    return row_layout(t, &rows, &stride) && stride == t->ne[0];
}

// fp32 vector of n contiguous elements whose single non-unit dim is `dim`.
bool is_vec(const dt_tensor* t, int64_t n, int dim = 0) {
    if (!t || !contiguous_f32(t)) return false;
    for (int i = 0; i < 4; ++i)
        if (t->ne[i] != (i == dim ? n : 1)) return false;
    return true;
}

enum Kind {
    K_NONE, K_ADALN, K_GATED, K_SWIGLU, K_GN, K_QK, K_SILU, K_GEMM_ADD, K_GEMM_GROUP, K_RES_ADALN, K_QK_SWIGLU,
    K_CONV, K_ATTN_QK, K_DEFERRED
};

struct QkSeg {
    const dt_tensor* q;   // RMS_NORM input
    const dt_tensor* w;   // norm weight [head_dim]
    int64_t tok0, tokens; // token range inside the rope output
    float eps;            // the RMS_NORM's eps
};

struct Plan {
    Kind kind = K_NONE;
    const dt_tensor* in[6] = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    float eps = 0.f;
    float addend = 0.f;  // adaLN: added to every scale (the 1 of 1 + scale)
    int silu = 0;
    int up2 = 0;  // CONV: the input is upsampled 2x (nearest) on the fly
    // CONV with a residual (in[4]): the output is res + conv, times
    // res_scale when res_scaled
    int res_scaled = 0;
    float res_scale = 1.f;
    // CONV with a GroupNorm (+ SiLU) of in[0] applied in its channel-last
    // copy: gn_groups > 0, the affine gn_w / gn_b (or null), eps and silu
    // in `eps` / `silu`
    int64_t gn_groups = 0;
    const dt_tensor* gn_w = nullptr;
    const dt_tensor* gn_b = nullptr;
    // QK
    std::vector<QkSeg> segs;
    std::vector<const dt_tensor*> pos;  // per axis
    int axis_dim = 0;
    float base = 0.f;
    // GEMM group: every member MUL_MAT, the root first
    std::vector<const dt_tensor*> members;
    // QK + SwiGLU: the k tensor's QK segment and root, the SwiGLU's inputs and root
    QkSeg kseg{};
    const dt_tensor* kroot = nullptr;
    const dt_tensor* sw[3] = {nullptr, nullptr, nullptr};  // gate, up, output
};

struct Graph {
    std::unordered_map<const dt_tensor*, int> uses;
    std::unordered_map<const dt_tensor*, int> index;
    std::vector<char> claimed;
    std::vector<int> root;   // index of the node whose fused kernel absorbs node i
    std::vector<int> runs_at;  // position where node i's kernel runs
    std::vector<char> deferred;  // node i keeps its output but runs inside another node's kernel
    std::unordered_map<const dt_tensor*, std::vector<int>> consumers;
    // Set by the memory-hazard check (check_plan_memory) for launches that
    // would read clobbered memory under the caller's allocation: `nomove`
    // keeps node i's launch at its own position and output set (no deferral,
    // grouping, merging or attention prologue rooted at or absorbing i);
    // `banned` also keeps i out of every fused kernel.
    std::vector<char> nomove, banned;
    dt_tensor** nodes = nullptr;
    int current_root = -1;

    bool internal(const dt_tensor* t, int n_uses = 1) const {
        if (!t || (t->flags & DT_FLAG_OUTPUT)) return false;
        auto i = index.find(t);
        if (i == index.end() || claimed[i->second] || banned[i->second]) return false;
        auto u = uses.find(t);
        return u != uses.end() && u->second == n_uses;
    }
    void claim(const dt_tensor* t) {
        const int i = index.at(t);
        claimed[i] = 1;
        root[i] = current_root;
    }
};

const dt_tensor* nodes_at(const Graph& g, int i) { return g.nodes[i]; }

// The modulation factor t = ADD(s, FILL(c)) of n * (1 + scale): s an fp32
// vector of `cols`, the scalar FILL of Tensor.hpp:233-236 (`1.0f + scale`
// becomes add(scale, full(1))), both used only here, possibly seen through a
// zero-offset VIEW of the same vector (AdaLayerNormContinuous.inl:30-40
// indexes (1 + scale)[:, None, :]).  The adaLN kernels add c to each scale
// as they stage it -- the ADD's own single fp32 rounding -- so the ADD and
// the FILL need no launches.  Otherwise t itself is the factor.
struct ScaleFactor {
    const dt_tensor* vec = nullptr;
    float addend = 0.f;
    const dt_tensor* add = nullptr;   // claimed with the plan
    const dt_tensor* fill = nullptr;
    const dt_tensor* view = nullptr;
};

bool scale_factor(Graph& g, const dt_tensor* t, int64_t cols, ScaleFactor* out) {
    *out = ScaleFactor{t, 0.f, nullptr, nullptr, nullptr};
    if (!is_vec(t, cols)) return false;
    const dt_tensor* view = nullptr;
    const dt_tensor* a = t;
    if (t->op == DT_OP_VIEW && view_offset(t) == 0 && g.internal(t)) {
        view = t;
        a = t->src[0];
    }
    if (a && a->op == DT_OP_ADD && is_vec(a, cols) && g.internal(a))
        for (int k = 0; k < 2; ++k) {
            const dt_tensor* v = a->src[k];
            const dt_tensor* f = a->src[1 - k];
            if (!f || f->op != DT_OP_FILL || f->type != DT_TYPE_F32 || !g.internal(f) ||
                f->ne[0] * f->ne[1] * f->ne[2] * f->ne[3] != 1 || !is_vec(v, cols))
                continue;
            *out = ScaleFactor{v, fparam(f, 0), a, f, view};
            return true;
        }
    return true;
}

void claim_factor(Graph& g, const ScaleFactor& f) {
    if (f.add) {
        if (f.view) g.claim(f.view);
        g.claim(f.add);
        g.claim(f.fill);
    }
}

bool match_adaln(Graph& g, const dt_tensor* a, Plan& p) {
    if (a->op != DT_OP_ADD) return false;
    const dt_tensor* m = a->src[0];
    const dt_tensor* sh = a->src[1];
    if (!m || m->op != DT_OP_MUL || !g.internal(m)) return false;
    const dt_tensor* n = m->src[0];
    const dt_tensor* t = m->src[1];
    if (!n || n->op != DT_OP_NORM || !g.internal(n)) return false;
    const dt_tensor* x = n->src[0];
    const int64_t cols = x->ne[0];
    int64_t r1, s1, r2, s2;
    ScaleFactor f;
    if (!scale_factor(g, t, cols, &f) || !is_vec(sh, cols) || !same_shape(x, a) || x->type != a->type ||
        !is_io_type(x->type) || !row_layout(x, &r1, &s1) || !row_layout(a, &r2, &s2))
        return false;
    g.claim(m);
    g.claim(n);
    claim_factor(g, f);
    p.kind = K_ADALN;
    p.in[0] = x;
    p.in[1] = f.vec;
    p.in[2] = sh;
    p.addend = f.addend;
    p.eps = fparam(n, 0);
    return true;
}

// Gated-residual operands of r = ADD(h, MUL(o, gate[c])) (either operand
// order), with the MUL used only there.
bool gated_parts(Graph& g, const dt_tensor* a, const dt_tensor** h_out, const dt_tensor** o_out,
                 const dt_tensor** gate_out, const dt_tensor** m_out) {
    if (a->op != DT_OP_ADD) return false;
    for (int k = 1; k >= 0; --k) {
        const dt_tensor* m = a->src[k];
        const dt_tensor* h = a->src[1 - k];
        if (!m || !h || m->op != DT_OP_MUL || !g.internal(m)) continue;
        const dt_tensor* o = m->src[0];
        const dt_tensor* gate = m->src[1];
        int64_t r, s;
        if (!is_vec(gate, a->ne[0]) || !same_shape(h, a) || !same_shape(o, a) ||
            h->type != a->type || o->type != a->type || !is_io_type(a->type) ||
            !row_layout(h, &r, &s) || !row_layout(o, &r, &s) || !row_layout(a, &r, &s))
            continue;
        *h_out = h;
        *o_out = o;
        *gate_out = gate;
        *m_out = m;
        return true;
    }
    return false;
}

// The adaLN chain ADD(MUL(NORM(r), t), shift) over a gated residual r that
// is stored (read again later): one kernel writes r and the normalised
// output at the adaLN's position.  Every other reader of r must come later.
bool match_res_adaln(Graph& g, const dt_tensor* a, Plan& p) {
    if (a->op != DT_OP_ADD) return false;
    const dt_tensor* m = a->src[0];
    const dt_tensor* sh = a->src[1];
    if (!m || m->op != DT_OP_MUL || !g.internal(m)) return false;
    const dt_tensor* n = m->src[0];
    const dt_tensor* t = m->src[1];
    if (!n || n->op != DT_OP_NORM || !g.internal(n)) return false;
    const dt_tensor* x = n->src[0];
    auto xi = g.index.find(x);
    if (xi == g.index.end() || g.claimed[xi->second] || g.deferred[xi->second] || g.nomove[xi->second] ||
        g.banned[xi->second] || g.nomove[g.current_root])
        return false;
    const int64_t cols = x->ne[0];
    int64_t r1, s1, r2, s2;
    ScaleFactor f;
    if (!scale_factor(g, t, cols, &f) || !is_vec(sh, cols) || !same_shape(x, a) || x->type != a->type ||
        !is_io_type(x->type) || !row_layout(x, &r1, &s1) || !row_layout(a, &r2, &s2))
        return false;
    const dt_tensor *h, *o, *gate, *gm;
    if (!gated_parts(g, x, &h, &o, &gate, &gm)) return false;
    for (int c : g.consumers[x])
        if (nodes_at(g, c) != n && c <= g.current_root) return false;
    g.claim(m);
    g.claim(n);
    g.claim(gm);
    claim_factor(g, f);
    g.deferred[xi->second] = 1;
    g.runs_at[xi->second] = g.current_root;
    p.kind = K_RES_ADALN;
    p.in[0] = h;
    p.in[1] = o;
    p.in[2] = gate;
    p.in[3] = x;
    p.in[4] = f.vec;
    p.in[5] = sh;
    p.addend = f.addend;
    p.eps = fparam(n, 0);
    return true;
}

bool match_gated(Graph& g, const dt_tensor* a, Plan& p) {
    if (a->op != DT_OP_ADD) return false;
    for (int k = 1; k >= 0; --k) {
        const dt_tensor* m = a->src[k];
        const dt_tensor* h = a->src[1 - k];
        if (!m || !h || m->op != DT_OP_MUL || !g.internal(m)) continue;
        const dt_tensor* o = m->src[0];
        const dt_tensor* gate = m->src[1];
        int64_t r, s;
        if (!is_vec(gate, a->ne[0]) || !same_shape(h, a) || !same_shape(o, a) ||
            h->type != a->type || o->type != a->type || !is_io_type(a->type) ||
            !row_layout(h, &r, &s) || !row_layout(o, &r, &s) || !row_layout(a, &r, &s))
            continue;
        g.claim(m);
        p.kind = K_GATED;
        p.in[0] = h;
        p.in[1] = o;
        p.in[2] = gate;
        return true;
    }
    return false;
}

bool match_swiglu(Graph& g, const dt_tensor* y, Plan& p) {
    if (y->op != DT_OP_MUL) return false;
    for (int k = 0; k < 2; ++k) {
        const dt_tensor* a = y->src[k];
        const dt_tensor* u = y->src[1 - k];
        if (!a || !u || a->op != DT_OP_MUL || !g.internal(a)) continue;
        for (int j = 0; j < 2; ++j) {
            const dt_tensor* gt = a->src[j];
            const dt_tensor* s = a->src[1 - j];
            if (!gt || !s || s->op != DT_OP_SIGMOID || s->src[0] != gt || !g.internal(s)) continue;
            int64_t r, st;
            if (!same_shape(gt, y) || !same_shape(u, y) || gt->type != y->type ||
                u->type != y->type || !is_io_type(y->type) || !row_layout(gt, &r, &st) ||
                !row_layout(u, &r, &st) || !row_layout(y, &r, &st))
                continue;
            g.claim(a);
            g.claim(s);
            p.kind = K_SWIGLU;
            p.in[0] = gt;
            p.in[1] = u;
            return true;
        }
    }
    return false;
}

// GroupNorm over x ne {W, H, C, N}: NORM of a VIEW with ne {C/G*H*W, G, N, 1},
// VIEWed back to x's shape, then optional MUL(w), ADD(b), SiLU.
bool match_groupnorm(Graph& g, const dt_tensor* root, Plan& p) {
    std::vector<std::pair<const dt_tensor*, int>> chain;  // interior node, expected uses
    const dt_tensor* cur = root;
    int silu = 0;
    if (root->op == DT_OP_MUL) {
        for (int k = 0; k < 2; ++k) {
            const dt_tensor* a = root->src[k];
            const dt_tensor* s = root->src[1 - k];
            if (a && s && s->op == DT_OP_SIGMOID && s->src[0] == a) {
                silu = 1;
                chain.push_back({s, 1});
                cur = a;
                break;
            }
        }
    }
    int cur_uses = silu ? 2 : 1;  // the SiLU input feeds both SIGMOID and the final MUL
    auto push = [&](const dt_tensor* t) {
        if (t != root) chain.push_back({t, cur_uses});
        cur_uses = 1;
    };
    const dt_tensor *w = nullptr, *b = nullptr;
    if (cur->op == DT_OP_ADD && cur->src[0] && cur->src[0]->op == DT_OP_MUL) {
        b = cur->src[1];
        push(cur);
        cur = cur->src[0];
    }
    if (cur->op == DT_OP_MUL && cur->src[0] && cur->src[0]->op == DT_OP_VIEW) {
        w = cur->src[1];
        push(cur);
        cur = cur->src[0];
    }
    if (cur->op != DT_OP_VIEW || !(silu || w || b)) return false;  // a bare norm runs unfused
    const dt_tensor* r = cur;
    push(r);
    const dt_tensor* n = r->src[0];
    if (!n || n->op != DT_OP_NORM) return false;
    push(n);
    const dt_tensor* v = n->src[0];
    if (!v || v->op != DT_OP_VIEW) return false;
    push(v);
    const dt_tensor* x = v->src[0];
    if (!x) return false;
    for (const auto& c : chain)
        if (!g.internal(c.first, c.second)) return false;
    // Shapes: x is contiguous NCHW = ne {W, H, C, N}; v is ne {L, G, N, 1}.
    const int64_t W_ = x->ne[0], H_ = x->ne[1], C = x->ne[2], N = x->ne[3];
    const int64_t G = v->ne[1];
    int64_t rows, stride;
    if (!is_io_type(x->type) || x->type != root->type || !same_shape(x, root) || G <= 0 ||
        C % G || v->ne[0] != C / G * H_ * W_ || v->ne[2] != N || v->ne[3] != 1 ||
        !row_layout(x, &rows, &stride) || stride != W_ || !row_layout(root, &rows, &stride) ||
        stride != W_ || view_offset(v) != 0 || view_offset(r) != 0 || !same_shape(r, x) ||
        v->nb[0] != elem_size(x->type) || v->nb[1] != v->ne[0] * v->nb[0] ||
        r->nb[0] != elem_size(x->type) || r->nb[1] != W_ * r->nb[0])
        return false;
    if ((w && !is_vec(w, C, 2)) || (b && !is_vec(b, C, 2))) return false;
    for (const auto& c : chain) g.claim(c.first);
    p.kind = K_GN;
    p.in[0] = x;
    p.in[1] = w;
    p.in[2] = b;
    p.in[3] = v;
    p.eps = fparam(n, 0);
    p.silu = silu;
    return true;
}

// FLASH_ATTN_EXT whose q is VIEW(y) with y's token and head axes swapped
// (the [B, S, H, D] -> ggml q layout of FlashAttentionOp.cpp:84-94) and y a
// BF16 QK-RMSNorm+RoPE root (match_qk) used only there: the chain becomes
// the attention's prologue.  One or two segments (txt | img, one eps),
// head_dim 128, axis_dim % 8 == 0; otherwise nothing is claimed.
bool match_qk(Graph& g, const dt_tensor* y, Plan& p);

bool match_attn_qk(Graph& g, const dt_tensor* t, Plan& p) {
    if (t->op != DT_OP_FLASH_ATTN_EXT || t->src[3] || t->type != DT_TYPE_BF16 || g.nomove[g.current_root])
        return false;
    const dt_tensor* qv = t->src[0];
    if (!qv || qv->op != DT_OP_VIEW || !g.internal(qv) || view_offset(qv) != 0) return false;
    const dt_tensor* y = qv->src[0];
    if (!y || y->op != DT_OP_CONCAT || y->type != DT_TYPE_BF16 || !g.internal(y) || g.nomove[g.index.at(y)])
        return false;
    if (qv->ne[0] != 128 || y->ne[0] != 128 || qv->ne[1] != y->ne[2] || qv->ne[2] != y->ne[1] ||
        qv->ne[3] != y->ne[3] || qv->nb[0] != 2 || qv->nb[1] != y->nb[2] || qv->nb[2] != y->nb[1])
        return false;
    const std::vector<char> claimed = g.claimed;
    const std::vector<int> root = g.root;
    Plan qp;
    bool ok = match_qk(g, y, qp) && qp.segs.size() <= 2 && qp.axis_dim % 8 == 0 &&
              (qp.segs.size() == 1 || qp.segs[0].eps == qp.segs[1].eps);
    for (const QkSeg& sg : qp.segs)
        ok = ok && sg.q->type == DT_TYPE_BF16 && sg.q->nb[1] % 16 == 0 && sg.q->nb[2] % 16 == 0;
    if (!ok) {
        g.claimed = claimed;
        g.root = root;
        return false;
    }
    g.claim(y);
    g.claim(qv);
    p = qp;
    p.kind = K_ATTN_QK;
    p.in[0] = qv;
    return true;
}

bool match_groupnorm(Graph& g, const dt_tensor* root, Plan& p);

// Conv2d::forward (Conv2d.cpp:38-102): CONV_2D_DIRECT, or ADD(conv, bias
// reshaped to [1, Co, 1, 1]) with the conv used only there.  An UPSCALE x2
// input used only by the conv (Upsample2D.cpp:50-72) is read through the
// conv's upsampled addressing instead of being materialised.  A 3x3 conv's
// input that is a GroupNorm (+ affine) (+ SiLU) chain read only here -- the
// norm -> SiLU -> conv of ResnetBlock2D.inl:114-127, 163-176 and the
// decoder's conv_out -- is normalised by the conv's channel-last copy, so
// the normalised tensor is never stored.  Operand checks happen at
// execution (run_conv), where a mismatch is reported.
bool match_conv(Graph& g, const dt_tensor* t, Plan& p) {
    const dt_tensor* c = nullptr;
    const dt_tensor* bias = nullptr;
    if (t->op == DT_OP_CONV_2D_DIRECT) {
        c = t;
    } else if (t->op == DT_OP_ADD) {
        for (int k = 0; k < 2 && !c; ++k) {
            const dt_tensor* a = t->src[k];
            const dt_tensor* b = t->src[1 - k];
            if (a && a->op == DT_OP_CONV_2D_DIRECT && g.internal(a) && same_shape(a, t) && a->type == t->type &&
                is_vec(b, a->ne[2], 2) && dense(t)) {
                c = a;
                bias = b;
            }
        }
    }
    if (!c || !c->src[0] || !c->src[1]) return false;
    const dt_tensor* x = c->src[1];
    const dt_tensor* up = nullptr;
    if (x->op == DT_OP_UPSCALE && x->op_params[0] == 2 && x->src[0] && g.internal(x) &&
        x->src[0]->type == x->type && dense(x->src[0])) {
        up = x;
        x = x->src[0];
    }
    if (c != t) g.claim(c);
    if (up) g.claim(up);
    Plan gp;
    const bool gn = c->src[0]->ne[0] == 3 && g.internal(x) && match_groupnorm(g, x, gp);
    if (gn) {
        g.claim(x);
        x = gp.in[0];
    }
    p.kind = K_CONV;
    p.in[0] = x;
    p.in[1] = c->src[0];
    p.in[2] = bias;
    p.in[3] = c;
    p.up2 = up != nullptr;
    if (gn) {
        p.gn_groups = gp.in[3]->ne[1];
        p.gn_w = gp.in[1];
        p.gn_b = gp.in[2];
        p.eps = gp.eps;
        p.silu = gp.silu;
    }
    return true;
}

// The tail of ResnetBlock2D::forward (ResnetBlock2D.inl:194): `(input +
// hidden) / output_scale_factor` records ADD(res, h) then SCALE(1 / f)
// (Tensor / float is ggml_scale); h is conv2's output, in one of
// match_conv's forms and used only by the ADD.  The conv's epilogue adds
// the residual and scales, with the ADD's value rounded to the node type
// as the graph stores it, so neither full-tensor pass runs.  Without the
// SCALE (a factor of 1 still records it; a graph may also end at the ADD)
// the ADD alone is folded.  When both operands are convs (a block with a
// 1x1 conv_shortcut), the 3x3 one takes the residual: its epilogue stages
// the output through LDS, where the 1x1 kernel's would load the residual
// element by element.  Among equals, hidden_states (the ADD's src1) does.
bool match_conv_residual(Graph& g, const dt_tensor* t, Plan& p) {
    const dt_tensor* add = t;
    if (t->op == DT_OP_SCALE) {
        add = t->src[0];
        if (!add || add->op != DT_OP_ADD || !g.internal(add) || !same_shape(add, t) || add->type != t->type ||
            fparam(t, 1) != 0.f)
            return false;
    }
    if (add->op != DT_OP_ADD || !dense(t)) return false;
    // the conv node under h (CONV_2D_DIRECT itself, or under its bias ADD)
    auto conv_of = [](const dt_tensor* h) -> const dt_tensor* {
        if (!h) return nullptr;
        if (h->op == DT_OP_CONV_2D_DIRECT) return h;
        if (h->op != DT_OP_ADD) return nullptr;
        for (int k = 0; k < 2; ++k)
            if (h->src[k] && h->src[k]->op == DT_OP_CONV_2D_DIRECT) return h->src[k];
        return nullptr;
    };
    auto is3x3 = [&](const dt_tensor* h) {
        const dt_tensor* c = conv_of(h);
        return c && c->src[0] && c->src[0]->ne[0] == 3;
    };
    int order[2] = {1, 0};
    if (!is3x3(add->src[1]) && is3x3(add->src[0])) {
        order[0] = 0;
        order[1] = 1;
    }
    for (int k : order) {
        const dt_tensor* h = add->src[k];
        const dt_tensor* res = add->src[1 - k];
        if (!h || !res || h == res || !g.internal(h) || !same_shape(h, add) || h->type != add->type ||
            !same_shape(res, add) || res->type != add->type || !dense(res))
            continue;
        if (!conv_of(h)) continue;
        Plan cp;
        if (!match_conv(g, h, cp)) continue;
        g.claim(h);
        if (add != t) g.claim(add);
        p = cp;
        p.in[4] = res;
        p.res_scaled = add != t;
        p.res_scale = add != t ? fparam(t, 0) : 1.0f;
        return true;
    }
    return false;
}

// MUL(x, SIGMOID(x)): the SiLU module's composite (SiLU.hpp:12) as one kernel.
bool match_silu(Graph& g, const dt_tensor* y, Plan& p) {
    if (y->op != DT_OP_MUL) return false;
    for (int k = 0; k < 2; ++k) {
        const dt_tensor* x = y->src[k];
        const dt_tensor* s = y->src[1 - k];
        if (x && s && s->op == DT_OP_SIGMOID && s->src[0] == x && g.internal(s) &&
            same_shape(x, y)) {
            g.claim(s);
            p.kind = K_SILU;
            p.in[0] = x;
            return true;
        }
    }
    return false;
}

// Leaves of a CONCAT tree along ne0, left to right.
bool concat_leaves(Graph& g, const dt_tensor* t, bool is_root, std::vector<const dt_tensor*>& out,
                   std::vector<const dt_tensor*>& chain) {
    if (t->op == DT_OP_CONCAT && t->op_params[0] == 0 && (is_root || g.internal(t))) {
        if (!is_root) chain.push_back(t);
        return concat_leaves(g, t->src[0], false, out, chain) &&
               concat_leaves(g, t->src[1], false, out, chain);
    }
    out.push_back(t);
    return true;
}

bool match_qk(Graph& g, const dt_tensor* y, Plan& p) {
    if (y->op != DT_OP_CONCAT) return false;
    std::vector<const dt_tensor*> leaves, chain;
    if (!concat_leaves(g, y, true, leaves, chain) || leaves.size() < 2 ||
        leaves.size() > (size_t)kMaxRopeAxes)
        return false;
    const int n_axes = (int)leaves.size();
    const dt_tensor* wsrc = nullptr;
    int axis_dim = 0;
    float base = 0.f;
    std::vector<const dt_tensor*> pos;
    for (int a = 0; a < n_axes; ++a) {
        const dt_tensor* r = leaves[a];
        if (r->op != DT_OP_ROPE || !g.internal(r)) return false;
        const dt_tensor* v = r->src[0];
        const dt_tensor* ps = r->src[1];
        if (!v || v->op != DT_OP_VIEW || !g.internal(v) || !ps || ps->type != DT_TYPE_I32) return false;
        const int nd = r->op_params[0];
        if (r->op_params[1] != 0 || fparam(r, 3) != 1.0f || fparam(r, 4) != 0.0f ||
            fparam(r, 5) != 1.0f || nd != v->ne[0])
            return false;
        if (a == 0) {
            wsrc = v->src[0];
            axis_dim = nd;
            base = fparam(r, 2);
        }
        if (v->src[0] != wsrc || nd != axis_dim || fparam(r, 2) != base) return false;
        const int es = elem_size(wsrc->type);
        if (view_offset(v) != (int64_t)a * axis_dim * es) return false;
        if (v->nb[0] != es) return false;
        for (int i = 1; i < 4; ++i)
            if (v->ne[i] != wsrc->ne[i] || v->nb[i] != wsrc->nb[i]) return false;
        if (ps->ne[0] != wsrc->ne[2] || ps->ne[1] != 1 || ps->ne[2] != 1 || ps->ne[3] != 1 ||
            ps->nb[0] % 4)
            return false;
        chain.push_back(r);
        chain.push_back(v);
        pos.push_back(ps);
    }
    if (!wsrc || !g.internal(wsrc, n_axes)) return false;
    const int64_t head_dim = wsrc->ne[0];
    if ((int64_t)n_axes * axis_dim != head_dim || !same_shape(wsrc, y) || y->ne[3] != 1 ||
        y->type != wsrc->type || !is_io_type(y->type) || y->nb[0] != elem_size(y->type))
        return false;
    // Segments: MUL(RMS_NORM(q), w) directly, or a CONCAT of two along ne2.
    std::vector<const dt_tensor*> muls;
    std::vector<int64_t> tok0;
    if (wsrc->op == DT_OP_CONCAT && wsrc->op_params[0] == 2) {
        muls = {wsrc->src[0], wsrc->src[1]};
        tok0 = {0, wsrc->src[0] ? wsrc->src[0]->ne[2] : 0};
    } else {
        muls = {wsrc};
        tok0 = {0};
    }
    std::vector<QkSeg> segs;
    for (size_t i = 0; i < muls.size(); ++i) {
        const dt_tensor* m = muls[i];
        if (!m || m->op != DT_OP_MUL) return false;
        if (m != wsrc && !g.internal(m)) return false;
        const dt_tensor* rn = m->src[0];
        const dt_tensor* w = m->src[1];
        if (!rn || rn->op != DT_OP_RMS_NORM || !g.internal(rn) || !is_vec(w, head_dim)) return false;
        const dt_tensor* q = rn->src[0];
        if (q->type != y->type || q->ne[0] != head_dim || q->ne[1] != y->ne[1] || q->ne[3] != 1 ||
            q->nb[0] != elem_size(q->type))
            return false;
        if (m != wsrc) chain.push_back(m);
        chain.push_back(rn);
        segs.push_back({q, w, tok0[i], q->ne[2], fparam(rn, 0)});
    }
    if (segs.back().tok0 + segs.back().tokens != y->ne[2]) return false;
    chain.push_back(wsrc);
    for (const dt_tensor* t : chain) g.claim(t);
    p.kind = K_QK;
    p.segs = segs;
    p.pos = pos;
    p.axis_dim = axis_dim;
    p.base = base;
    return true;
}

// Operands of MUL_MAT node t as a dt_gemm_bf16 / dt_gemm_q8_0 call: weight
// rows [N][K] (BF16, or a whole DT_TYPE_Q8_0_SPLIT weight: codes, then
// scales bs [K/32][N]), activation rows [M][K], output rows [M][N].
struct GemmArgs {
    const void *a, *b;
    int64_t lda, ldb, M, N, K;
    const float* bs;
    int64_t ldbs;
    bool f32;  // F32 weight and activation: the fp32 GEMM
};

bool q8_weight(const dt_tensor* t) { return t->src[0] && t->src[0]->type == DT_TYPE_Q8_0_SPLIT; }

bool f32_gemm(const dt_tensor* t) {
    return t->src[0] && t->src[1] && t->src[0]->type == DT_TYPE_F32 && t->src[1]->type == DT_TYPE_F32;
}

bool gemm_args(const dt_tensor* t, GemmArgs* g) {
    const dt_tensor* w = t->src[0];
    const dt_tensor* x = t->src[1];
    if (!w || !x) return false;
    g->f32 = f32_gemm(t);
    if (g->f32) {
        if (t->type != DT_TYPE_F32 || w->ne[2] != 1 || w->ne[3] != 1 || x->ne[0] != w->ne[0] || w->nb[0] != 4 ||
            (w->ne[1] > 1 && w->nb[1] % 4))
            return false;
        int64_t rows, xs;
        if (!row_layout(x, &rows, &xs)) return false;
        *g = GemmArgs{x->data, w->data, xs, w->ne[1] > 1 ? w->nb[1] / 4 : w->ne[0], rows, w->ne[1], w->ne[0],
                      nullptr, 0, true};
        return true;
    }
    if (x->type != DT_TYPE_BF16) return false;
    const bool q8 = w->type == DT_TYPE_Q8_0_SPLIT;
    if (!q8 && w->type != DT_TYPE_BF16) return false;
    if (w->ne[2] != 1 || w->ne[3] != 1 || x->ne[0] != w->ne[0]) return false;
    if (q8) {
        // The scales sit after all N rows of codes: only the whole weight.
        if (w->op == DT_OP_VIEW || w->nb[0] != 1 || (w->ne[1] > 1 && w->nb[1] != w->ne[0])) return false;
    } else if (w->nb[0] != 2 || (w->ne[1] > 1 && w->nb[1] % 2)) {
        return false;
    }
    int64_t rows, xs;
    if (!row_layout(x, &rows, &xs)) return false;
    g->a = x->data;
    g->lda = xs;
    g->b = w->data;
    g->M = rows;
    g->N = w->ne[1];
    g->K = w->ne[0];
    if (q8) {
        g->ldb = g->K;
        g->bs = w->data ? reinterpret_cast<const float*>((const char*)w->data +
                                                         dt_q8_0_split_scale_offset(g->N, g->K))
                        : nullptr;
        g->ldbs = g->N;
    } else {
        g->ldb = w->ne[1] > 1 ? w->nb[1] / 2 : w->ne[0];
        g->bs = nullptr;
        g->ldbs = 0;
    }
    return true;
}

bool out_rows(const dt_tensor* t, int64_t n_cols, int64_t* ld) {
    int64_t rows;
    return (t->type == DT_TYPE_BF16 || t->type == DT_TYPE_F32) && t->ne[0] == n_cols &&
           row_layout(t, &rows, ld);
}

// ADD(y, MUL_MAT(w, x)) or ADD(MUL_MAT(w, x), y) -> one GEMM with addend y.
bool match_gemm_add(Graph& g, const dt_tensor* a, Plan& p) {
    if (a->op != DT_OP_ADD) return false;
    for (int k = 1; k >= 0; --k) {
        const dt_tensor* mm = a->src[k];
        const dt_tensor* y = a->src[1 - k];
        if (!mm || !y || mm->op != DT_OP_MUL_MAT || !g.internal(mm)) continue;
        int64_t ld;
        if (!same_shape(mm, a) || !same_shape(y, a) || y->type != a->type || mm->type != a->type ||
            !out_rows(a, a->ne[0], &ld) || !out_rows(y, a->ne[0], &ld))
            continue;
        g.claim(mm);
        p.kind = K_GEMM_ADD;
        p.in[0] = mm;
        p.in[1] = y;
        return true;
    }
    return false;
}

constexpr const char* kMulMatOperands =
    "dt_graph_compute: MUL_MAT needs BF16 or whole Q8_0_SPLIT weight rows and BF16 activation rows, or F32 "
    "weight and activation rows";

int run_mul_mat(dt_backend* be, const dt_tensor* mm, const dt_tensor* out, const dt_tensor* addend) {
    hipStream_t st = backend_stream(be);
    GemmArgs g;
    int64_t ldc = 0, ldd = 0;
    DT_REQUIRE(gemm_args(mm, &g), "%s", kMulMatOperands);
    DT_REQUIRE(out_rows(out, g.N, &ldc), "dt_graph_compute: MUL_MAT output must be BF16/F32 rows of N");
    if (addend) DT_REQUIRE(out_rows(addend, g.N, &ldd), "dt_graph_compute: bad GEMM addend");
    if (g.f32) {
        DT_REQUIRE(out->type == DT_TYPE_F32 && (!addend || addend->type == DT_TYPE_F32),
                   "dt_graph_compute: an F32 MUL_MAT writes F32");
        return dt_gemm_f32((const float*)g.a, g.lda, (const float*)g.b, g.ldb, (float*)out->data, ldc, g.M, g.N, g.K,
                           nullptr, addend ? (const float*)addend->data : nullptr, ldd, st);
    }
    if (g.bs)
        return dt_gemm_q8_0(g.a, g.lda, g.b, g.ldb, g.bs, g.ldbs, out->data, ldc, g.M, g.N, g.K, nullptr,
                            addend ? addend->data : nullptr, ldd, out->type, st);
    return dt_gemm_bf16(g.a, g.lda, g.b, g.ldb, out->data, ldc, g.M, g.N, g.K, nullptr,
                        addend ? addend->data : nullptr, ldd, out->type, st);
}

// Data address of t, resolving VIEW chains (a VIEW's own data is set only
// when the executor reaches it, which a grouped launch may precede).
const void* data_of(const dt_tensor* t) {
    int64_t off = 0;
    while (t && t->op == DT_OP_VIEW) {
        off += view_offset(t);
        t = t->src[0];
    }
    return t && t->data ? (const char*)t->data + off : nullptr;
}

// Independent MUL_MATs at one position: one grouped MFMA launch, whose
// tiles share the grid.
int run_gemm_group(dt_backend* be, const std::vector<const dt_tensor*>& members) {
    hipStream_t st = backend_stream(be);
    dt_gemm_problem ps[8];
    const int n = (int)members.size();
    DT_REQUIRE(n >= 1 && n <= 8, "dt_graph_compute: GEMM group of %d", n);
    GemmArgs gs[8];
    bool f32 = false;
    for (int i = 0; i < n; ++i) {
        const dt_tensor* mm = members[i];
        GemmArgs& g = gs[i];
        int64_t ldc = 0;
        DT_REQUIRE(gemm_args(mm, &g), "%s", kMulMatOperands);
        DT_REQUIRE(out_rows(mm, g.N, &ldc), "dt_graph_compute: MUL_MAT output must be BF16/F32 rows of N");
        g.a = data_of(mm->src[1]);
        g.b = data_of(mm->src[0]);
        if (g.bs) g.bs = reinterpret_cast<const float*>((const char*)g.b + dt_q8_0_split_scale_offset(g.N, g.K));
        ps[i] = dt_gemm_problem{g.a, g.lda, g.b, g.ldb, mm->data, ldc, nullptr, 0, nullptr, g.M, g.N, g.K, g.bs,
                                g.ldbs};
        DT_REQUIRE(i == 0 || g.f32 == f32, "dt_graph_compute: a GEMM group mixes F32 and BF16 products");
        f32 = g.f32;
    }
    if (f32) return dt_gemm_f32_grouped(ps, n, st);
    return dt_gemm_bf16_grouped(ps, n, members[0]->type, -1, st);
}

// Forward pass over unfused MUL_MATs: node i starts a group of the MUL_MATs
// that follow it with only VIEWs in between, whose inputs all run before i
// and whose output type and weight kind (BF16 or Q8_0_SPLIT) match; the later
// members run in i's launch.
void group_gemms(Graph& g, dt_tensor** nodes, int n, std::vector<Plan>& plans) {
    auto ready_before = [&](const dt_tensor* t, int pos) {
        while (t && t->op == DT_OP_VIEW) t = t->src[0];
        if (!t) return false;
        auto it = g.index.find(t);
        return it == g.index.end() || g.runs_at[it->second] < pos;
    };
    auto groupable = [&](int j) {
        const dt_tensor* t = nodes[j];
        GemmArgs ga;
        return t->op == DT_OP_MUL_MAT && !g.claimed[j] && !g.nomove[j] && !g.banned[j] && plans[j].kind == K_NONE &&
               gemm_args(t, &ga);
    };
    for (int i = 0; i < n; ++i) {
        if (!groupable(i) || !ready_before(nodes[i]->src[0], i) || !ready_before(nodes[i]->src[1], i)) continue;
        std::vector<int> members = {i};
        for (int j = i + 1; j < n && members.size() < 8; ++j) {
            const dt_tensor* t = nodes[j];
            if (t->op == DT_OP_VIEW) continue;
            if (!groupable(j) || t->type != nodes[i]->type || q8_weight(t) != q8_weight(nodes[i]) ||
                f32_gemm(t) != f32_gemm(nodes[i]) ||
                !ready_before(t->src[0], i) || !ready_before(t->src[1], i))
                break;
            members.push_back(j);
        }
        if (members.size() < 2) continue;
        Plan& p = plans[i];
        p.kind = K_GEMM_GROUP;
        p.members.clear();
        for (int j : members) {
            p.members.push_back(nodes[j]);
            if (j != i) {
                plans[j].kind = K_DEFERRED;
                g.runs_at[j] = i;
            }
        }
        i = members.back();
    }
}

// 256 x 256 tiles of a MUL_MAT (the GEMM's large tiles) and the waves of them
// one launch needs on MI355X's 256 CUs.  A planning estimate only (the plan
// is made without a device); the GEMM picks its tiles at launch.
int64_t big_tiles(const dt_tensor* t) {
    GemmArgs ga;
    if (!gemm_args(t, &ga)) return 0;
    return ((ga.M + 255) / 256) * ((ga.N + 255) / 256);
}
constexpr int64_t kPlanCus = 256;
int64_t tile_waves(int64_t tiles) { return (tiles + kPlanCus - 1) / kPlanCus; }

// Forward pass over the MUL_MATs still launched on their own: one whose
// output is first read after a later MUL_MAT launch of the same K, output
// type and weight kind runs in that launch when the two together take fewer
// waves of tiles than apart.  In a double-stream block the image
// feed-forward's output projection (4096 x 3072 x 9216, 192 tiles) is read
// only by its gated residual, which runs in the next block's adaLN, so it
// joins the text stream's (512 x 3072 x 9216, 24 tiles): one wave of 216
// instead of two launches.  The later launch keeps its position; the moved
// node's inputs stay alive until then (runs_at).
void defer_gemms(Graph& g, dt_tensor** nodes, int n, std::vector<Plan>& plans) {
    auto movable = [&](int j) {
        const dt_tensor* t = nodes[j];
        GemmArgs ga;
        return t->op == DT_OP_MUL_MAT && !g.claimed[j] && !g.nomove[j] && !g.banned[j] && plans[j].kind == K_NONE &&
               !(t->flags & DT_FLAG_OUTPUT) && gemm_args(t, &ga);
    };
    // The earliest launch position that reads t's value (through VIEWs).
    std::function<int(const dt_tensor*)> first_read = [&](const dt_tensor* t) {
        int first = n;
        auto it = g.consumers.find(t);
        if (it == g.consumers.end()) return first;
        for (int c : it->second) {
            if (nodes[c]->op == DT_OP_VIEW) {
                if (nodes[c]->flags & DT_FLAG_OUTPUT) return -1;
                first = std::min(first, first_read(nodes[c]));
            } else {
                first = std::min(first, g.runs_at[c]);
            }
        }
        return first;
    };
    for (int i = 0; i < n; ++i) {
        if (!movable(i)) continue;
        const dt_tensor* t = nodes[i];
        const int64_t K = t->src[0]->ne[0], ti = big_tiles(t);
        const int until = first_read(t);
        for (int j = i + 1; j < until; ++j) {
            const bool single = movable(j);
            const bool group = plans[j].kind == K_GEMM_GROUP && !g.nomove[j] && plans[j].members.size() < 8;
            if (!single && !group) continue;
            std::vector<const dt_tensor*> ms = group ? plans[j].members : std::vector<const dt_tensor*>{nodes[j]};
            bool fits = true;
            int64_t tj = 0, wj = 0;
            for (const dt_tensor* m : ms) {
                fits = fits && m->type == t->type && q8_weight(m) == q8_weight(t) && f32_gemm(m) == f32_gemm(t) &&
                       m->src[0]->ne[0] == K;
                tj += big_tiles(m);
            }
            wj = tile_waves(tj);
            if (!fits || tile_waves(ti + tj) >= tile_waves(ti) + wj) continue;
            Plan& p = plans[j];
            if (single) {
                p.kind = K_GEMM_GROUP;
                p.members = {nodes[j]};
            }
            p.members.push_back(t);
            plans[i].kind = K_DEFERRED;
            g.runs_at[i] = j;
            break;
        }
    }
}

// Forward pass over SwiGLU roots: with the two single-segment QK roots that
// precede it (q and k of the same block) and inputs computed before the
// first of them, the three run as one launch at the first QK's position
// (dt_qk_rmsnorm_rope_swiglu).  The other two roots keep their outputs.
// When the block's q went into its attention (K_ATTN_QK), the nearest QK
// root (k) and the SwiGLU run as one launch at the QK's position.
void merge_qk_swiglu(Graph& g, dt_tensor** nodes, int n, std::vector<Plan>& plans) {
    auto ready_before = [&](const dt_tensor* t, int pos) {
        while (t && t->op == DT_OP_VIEW) t = t->src[0];
        if (!t) return false;
        auto it = g.index.find(t);
        return it == g.index.end() || g.runs_at[it->second] < pos;
    };
    auto move_to = [&](int root, int pos) {
        plans[root].kind = K_DEFERRED;
        g.runs_at[root] = pos;
        for (int i = 0; i < n; ++i)
            if (g.claimed[i] && g.root[i] == root) g.runs_at[i] = pos;
    };
    for (int sidx = 0; sidx < n; ++sidx) {
        if (plans[sidx].kind != K_SWIGLU || g.nomove[sidx]) continue;
        int qk[2] = {-1, -1};
        int found = 0;
        for (int j = sidx - 1; j >= 0 && found < 2; --j)
            if (plans[j].kind == K_QK) qk[found++] = j;
        if (found == 0 || g.nomove[qk[0]]) continue;
        if (found == 2 && g.nomove[qk[1]]) found = 1;
        const Plan& S = plans[sidx];
        const dt_tensor* ys = nodes[sidx];
        auto merge_one = [&]() {  // the nearest QK root alone with the SwiGLU
            Plan& B = plans[qk[0]];
            if (B.segs.size() != 1 || nodes[qk[0]]->type != ys->type || !ready_before(S.in[0], qk[0]) ||
                !ready_before(S.in[1], qk[0]))
                return;
            B.kind = K_QK_SWIGLU;
            B.kroot = nullptr;
            B.sw[0] = S.in[0];
            B.sw[1] = S.in[1];
            B.sw[2] = ys;
            move_to(sidx, qk[0]);
        };
        if (found < 2) {
            merge_one();
            continue;
        }
        const int qa = qk[1], qb = qk[0];  // qa first in order
        Plan& A = plans[qa];
        Plan& B = plans[qb];
        const dt_tensor* ya = nodes[qa];
        const dt_tensor* yb = nodes[qb];
        if (A.segs.size() != 1 || B.segs.size() != 1 || A.pos != B.pos || A.axis_dim != B.axis_dim ||
            A.base != B.base || A.segs[0].eps != B.segs[0].eps || ya->type != yb->type || ys->type != ya->type) {
            merge_one();
            continue;
        }
        const dt_tensor* qa_in = A.segs[0].q;
        const dt_tensor* qb_in = B.segs[0].q;
        bool same = true;
        for (int d = 0; d < 4; ++d)
            same = same && qa_in->ne[d] == qb_in->ne[d] && qa_in->nb[d] == qb_in->nb[d] && ya->nb[d] == yb->nb[d] &&
                   ya->ne[d] == yb->ne[d];
        if (!same || !ready_before(qb_in, qa) || !ready_before(B.segs[0].w, qa) || !ready_before(S.in[0], qa) ||
            !ready_before(S.in[1], qa)) {
            merge_one();
            continue;
        }
        A.kind = K_QK_SWIGLU;
        A.kseg = B.segs[0];
        A.kroot = yb;
        A.sw[0] = S.in[0];
        A.sw[1] = S.in[1];
        A.sw[2] = ys;
        move_to(qb, qa);
        move_to(sidx, qa);
    }
}

// FLASH_ATTN_EXT with F32 q, k, v (and output): the fp32 attention, its
// scores in the backend's scratch.
int run_flash_attn_f32(dt_backend* be, const dt_tensor* t) {
    const dt_tensor *q = t->src[0], *k = t->src[1], *v = t->src[2];
    DT_REQUIRE(t->type == DT_TYPE_F32 && k->type == DT_TYPE_F32 && v->type == DT_TYPE_F32,
               "dt_graph_compute: FLASH_ATTN_EXT mixes F32 and other operand types");
    DT_REQUIRE(q->nb[0] == 4 && k->nb[0] == 4 && v->nb[0] == 4 && t->nb[0] == 4,
               "dt_graph_compute: FLASH_ATTN_EXT rows must be contiguous");
    DT_REQUIRE(t->ne[0] == q->ne[0] && t->ne[1] == q->ne[2] && t->ne[2] == q->ne[1] &&
                   t->ne[3] == q->ne[3] && k->ne[1] == v->ne[1] && k->ne[2] == q->ne[2] &&
                   v->ne[2] == q->ne[2] && k->ne[3] == q->ne[3] && v->ne[3] == q->ne[3] &&
                   k->ne[0] == q->ne[0] && v->ne[0] == q->ne[0],
               "dt_graph_compute: FLASH_ATTN_EXT shapes disagree");
    const int64_t qs[3] = {q->nb[3] / 4, q->nb[1] / 4, q->nb[2] / 4};
    const int64_t ks[3] = {k->nb[3] / 4, k->nb[1] / 4, k->nb[2] / 4};
    const int64_t vs[3] = {v->nb[3] / 4, v->nb[1] / 4, v->nb[2] / 4};
    const int64_t os[3] = {t->nb[3] / 4, t->nb[2] / 4, t->nb[1] / 4};
    const size_t ws_bytes = dt_flash_attn_f32_workspace_bytes(q->ne[3], q->ne[2], q->ne[1], k->ne[1], q->ne[0]);
    void* ws = nullptr;
    const int rc = backend_scratch(be, ws_bytes, &ws);
    if (rc) return rc;
    return dt_flash_attn_f32((const float*)q->data, (const float*)k->data, (const float*)v->data, (float*)t->data,
                             q->ne[3], q->ne[2], q->ne[1], k->ne[1], q->ne[0], qs, ks, vs, os, fparam(t, 0), ws,
                             ws_bytes, backend_stream(be));
}

int run_flash_attn(hipStream_t st, const dt_tensor* t) {
    const dt_tensor *q = t->src[0], *k = t->src[1], *v = t->src[2];
    DT_REQUIRE(q && k && v && !t->src[3], "dt_graph_compute: FLASH_ATTN_EXT needs q, k, v and no mask");
    DT_REQUIRE(q->type == DT_TYPE_BF16 && k->type == DT_TYPE_BF16 && v->type == DT_TYPE_BF16,
               "dt_graph_compute: FLASH_ATTN_EXT operands must be BF16");
    DT_REQUIRE(q->nb[0] == 2 && k->nb[0] == 2 && v->nb[0] == 2 && t->nb[0] == elem_size(t->type),
               "dt_graph_compute: FLASH_ATTN_EXT rows must be contiguous");
    DT_REQUIRE(t->ne[0] == q->ne[0] && t->ne[1] == q->ne[2] && t->ne[2] == q->ne[1] &&
                   t->ne[3] == q->ne[3] && k->ne[1] == v->ne[1] && k->ne[2] == q->ne[2] &&
                   v->ne[2] == q->ne[2] && k->ne[3] == q->ne[3] && v->ne[3] == q->ne[3] &&
                   k->ne[0] == q->ne[0] && v->ne[0] == q->ne[0],
               "dt_graph_compute: FLASH_ATTN_EXT shapes disagree");
    const int64_t es = elem_size(t->type);
    const int64_t qs[3] = {q->nb[3] / 2, q->nb[1] / 2, q->nb[2] / 2};
    const int64_t ks[3] = {k->nb[3] / 2, k->nb[1] / 2, k->nb[2] / 2};
    const int64_t vs[3] = {v->nb[3] / 2, v->nb[1] / 2, v->nb[2] / 2};
    const int64_t os[3] = {t->nb[3] / es, t->nb[2] / es, t->nb[1] / es};
    return dt_flash_attn_bf16(q->data, k->data, v->data, t->data, q->ne[3], q->ne[2], q->ne[1], k->ne[1],
                              q->ne[0], qs, ks, vs, os, fparam(t, 0), t->type, st);
}

// One convolution: F32 / BF16 weights packed into the backend's scratch
// (bf16 [Co][K*K][Ci] tiles; a few MB, re-packed per call) unless they come
// packed once at load (DT_TYPE_CONV2D_PACKED), the channel-last copy of x
// after them, then dt_conv2d into root.
// A CONV_2D_DIRECT (x, w, the bias or null, the conv node; up2: x is read
// 2x upsampled) writing root, with the plan's folds when `p` is given: the
// residual ADD / SCALE of in[4] and the GroupNorm of x (gn_groups > 0).
int run_conv(dt_backend* be, const dt_tensor* root, const dt_tensor* x, const dt_tensor* w, const dt_tensor* bias,
             const dt_tensor* conv, int up2, const Plan* p = nullptr) {
    hipStream_t st = backend_stream(be);
    const int64_t K = w->ne[0], Ci = w->ne[2], Co = w->ne[3];
    const int64_t W = x->ne[0], H = x->ne[1], N = x->ne[3], f = up2 ? 2 : 1;
    const int32_t* prm = conv->op_params;
    DT_REQUIRE(prm[0] == 1 && prm[1] == 1 && prm[4] == 1 && prm[5] == 1,
               "dt_graph_compute: CONV_2D_DIRECT with stride %d,%d / dilation %d,%d (1 only)", prm[0], prm[1],
               prm[4], prm[5]);
    DT_REQUIRE((K == 1 || K == 3) && w->ne[1] == K && prm[2] == (K - 1) / 2 && prm[3] == (K - 1) / 2,
               "dt_graph_compute: CONV_2D_DIRECT needs a square 1x1 / 3x3 kernel with padding (K - 1) / 2");
    const bool prepacked = w->type == DT_TYPE_CONV2D_PACKED;
    DT_REQUIRE(w->type == DT_TYPE_F32 || w->type == DT_TYPE_BF16 || prepacked,
               "dt_graph_compute: CONV_2D_DIRECT weight type %d", w->type);
    DT_REQUIRE(is_io_type(x->type) && x->type == root->type, "dt_graph_compute: CONV_2D_DIRECT input/output types");
    DT_REQUIRE(dense(x) && (prepacked || dense(w)) && dense(root),
               "dt_graph_compute: CONV_2D_DIRECT operands must be contiguous");
    DT_REQUIRE(x->ne[2] == Ci && root->ne[0] == W * f && root->ne[1] == H * f && root->ne[2] == Co &&
                   root->ne[3] == N,
               "dt_graph_compute: CONV_2D_DIRECT shapes disagree");
    const dt_tensor* res = p ? p->in[4] : nullptr;
    const int64_t G = p ? p->gn_groups : 0;
    DT_REQUIRE(!G || (K == 3 && Ci % G == 0), "dt_graph_compute: GroupNorm folded into a conv needs a 3x3 kernel");
    // Scratch: [packed weights][channel-last copy][GroupNorm partials][(mean, rstd)]
    const size_t packed = prepacked ? 0 : (dt_conv2d_packed_bytes(Co, Ci, K) + 255) / 256 * 256;
    const size_t ws = (dt_conv2d_workspace_bytes(N, Ci, H, W) + 255) / 256 * 256;
    const size_t gws = G ? (dt_groupnorm_workspace_bytes(N, Ci, H * W, G) + 255) / 256 * 256 : 0;
    const size_t mrb = G ? (size_t)(N * G) * sizeof(float2) : 0;
    void* scratch = nullptr;
    if (packed + ws + gws + mrb) {
        const int rc = backend_scratch(be, packed + ws + gws + mrb, &scratch);
        if (rc) return rc;
    }
    const void* wp = prepacked ? data_of(w) : scratch;
    if (!prepacked) {
        const int rc = dt_conv2d_pack_weights(data_of(w), w->type, Co, Ci, K, scratch, st);
        if (rc) return rc;
    }
    g_kernels += (prepacked ? 0 : 1) + (conv_uses_dma(K, root->type) ? 1 : 0) + 1;  // pack, channel-last copy, conv
    const float* b = bias ? (const float*)data_of(bias) : nullptr;
    void* wsp = ws ? (char*)scratch + packed : nullptr;
    if (!res && !G) return dt_conv2d(data_of(x), N, Ci, H, W, wp, Co, K, up2, b, root->data, wsp, ws, root->type, st);
    ConvFold fold;
    if (G) {
        float2* mr = (float2*)((char*)scratch + packed + ws + gws);
        g_kernels += 2;  // GroupNorm partials, (mean, rstd)
        const int rc = gn_mean_rstd(data_of(x), N, Ci, H * W, G, p->eps, (char*)scratch + packed + ws, mr, x->type, st);
        if (rc) return rc;
        fold.gn_mr = mr;
        fold.gn_w = p->gn_w ? (const float*)data_of(p->gn_w) : nullptr;
        fold.gn_b = p->gn_b ? (const float*)data_of(p->gn_b) : nullptr;
        fold.gn_groups = (int)G;
        fold.gn_silu = p->silu;
    }
    if (res) {
        // Each output element's residual is read by the thread that then
        // writes it, so the residual may be the output's own memory, but no
        // other part of it.
        const size_t bytes = (size_t)(N * Co * H * f * W * f) * (size_t)elem_size(root->type);
        const char* r = (const char*)data_of(res);
        const char* y = (const char*)root->data;
        DT_REQUIRE(same_shape(res, root) && res->type == root->type && dense(res),
                   "dt_graph_compute: the conv residual must match the output");
        DT_REQUIRE(r == y || r + bytes <= y || y + bytes <= r,
                   "dt_graph_compute: the conv residual partly overlaps the output");
        fold.res = r;
        fold.res_mode = p->res_scaled ? 2 : 1;
        fold.res_scale = p->res_scale;
    }
    return conv2d_fold(data_of(x), N, Ci, H, W, wp, Co, K, up2, b, fold, root->data, wsp, ws, root->type, st);
}

int run_upscale(hipStream_t st, const dt_tensor* t) {
    const dt_tensor* x = t->src[0];
    const int f = t->op_params[0];
    DT_REQUIRE(x && x->type == t->type && is_io_type(t->type) && dense(x) && dense(t),
               "dt_graph_compute: UPSCALE operands must be contiguous F32 / BF16 of one type");
    DT_REQUIRE(f >= 1 && t->ne[0] == x->ne[0] * f && t->ne[1] == x->ne[1] * f && t->ne[2] == x->ne[2] &&
                   t->ne[3] == x->ne[3],
               "dt_graph_compute: UPSCALE shapes disagree");
    return dt_op_upscale_nearest(data_of(x), x->ne[3], x->ne[2], x->ne[1], x->ne[0], f, t->data, t->type, st);
}

// FLASH_ATTN_EXT t with its q chain as the prologue (match_attn_qk): the
// segments' pre-norm q, norm weights and eps, the positions of the joint
// sequence, and the backend's device-built RoPE table, whose entries are
// the bits the QK kernels compute without a table.
int run_attn_qk(dt_backend* be, const dt_tensor* t, const Plan& p) {
    const dt_tensor *qv = p.in[0], *k = t->src[1], *v = t->src[2];
    DT_REQUIRE(k && v && k->type == DT_TYPE_BF16 && v->type == DT_TYPE_BF16 && k->nb[0] == 2 && v->nb[0] == 2 &&
                   t->nb[0] == elem_size(t->type),
               "dt_graph_compute: FLASH_ATTN_EXT k / v must be BF16 with contiguous rows");
    DT_REQUIRE(t->ne[0] == 128 && t->ne[1] == qv->ne[2] && t->ne[2] == qv->ne[1] && t->ne[3] == qv->ne[3] &&
                   k->ne[1] == v->ne[1] && k->ne[2] == qv->ne[2] && v->ne[2] == qv->ne[2] && k->ne[3] == qv->ne[3] &&
                   v->ne[3] == qv->ne[3] && k->ne[0] == 128 && v->ne[0] == 128,
               "dt_graph_compute: FLASH_ATTN_EXT shapes disagree");
    AttnQk qk{};
    for (size_t i = 0; i < p.segs.size(); ++i) {
        const dt_tensor* q = p.segs[i].q;
        qk.q[i] = data_of(q);
        qk.qs[i][0] = q->nb[3] / 2;
        qk.qs[i][1] = q->nb[2] / 2;
        qk.qs[i][2] = q->nb[1] / 2;
        qk.w[i] = (const float*)data_of(p.segs[i].w);
    }
    qk.split = p.segs.size() == 2 ? p.segs[1].tok0 : qv->ne[1];
    qk.eps = p.segs[0].eps;
    qk.n_axes = (int)p.pos.size();
    for (int a = 0; a < qk.n_axes; ++a) {
        qk.pos.stride[a] = p.pos[a]->nb[0] / 4;
        qk.pos.ptr[a] = (const int32_t*)data_of(p.pos[a]);
    }
    qk.axis_dim = p.axis_dim;
    qk.freq_base = p.base;
    int rc = backend_rope_table(be, p.axis_dim, p.base, &qk.table);
    if (rc) return rc;
    qk.n_pos = kBackendRopePositions;
    const int64_t es = elem_size(t->type);
    const int64_t ks[3] = {k->nb[3] / 2, k->nb[1] / 2, k->nb[2] / 2};
    const int64_t vs[3] = {v->nb[3] / 2, v->nb[1] / 2, v->nb[2] / 2};
    const int64_t os[3] = {t->nb[3] / es, t->nb[2] / es, t->nb[1] / es};
    return flash_attn_qk_launch(qk, k->data, v->data, t->data, qv->ne[3], qv->ne[2], qv->ne[1], k->ne[1], ks, vs,
                                os, fparam(t, 0), t->type, backend_stream(be));
}

int run_plan(dt_backend* be, const dt_tensor* root, Plan& p) {
    hipStream_t st = backend_stream(be);
    switch (p.kind) {
        case K_ADALN: {
            int64_t rows, xs, ys;
            row_layout(p.in[0], &rows, &xs);
            row_layout(root, &rows, &ys);
            ++g_kernels;
            return adaln_launch(p.in[0]->data, rows, root->ne[0], xs, (const float*)data_of(p.in[2]),
                                (const float*)data_of(p.in[1]), p.addend, root->data, ys, p.eps,
                                root->type, st);
        }
        case K_GATED: {
            int64_t rows, hs, os, ys;
            row_layout(p.in[0], &rows, &hs);
            row_layout(p.in[1], &rows, &os);
            row_layout(root, &rows, &ys);
            ++g_kernels;
            return dt_gated_residual(p.in[0]->data, hs, p.in[1]->data, os, (const float*)p.in[2]->data,
                                     root->data, ys, rows, root->ne[0], root->type, st);
        }
        case K_SWIGLU: {
            int64_t rows, gs, us, ys;
            row_layout(p.in[0], &rows, &gs);
            row_layout(p.in[1], &rows, &us);
            row_layout(root, &rows, &ys);
            ++g_kernels;
            return dt_swiglu(p.in[0]->data, gs, p.in[1]->data, us, root->data, ys, rows, root->ne[0],
                             root->type, st);
        }
        case K_GN: {
            const dt_tensor* x = p.in[0];
            const int64_t N = x->ne[3], C = x->ne[2], HW = x->ne[0] * x->ne[1], G = p.in[3]->ne[1];
            const size_t ws_bytes = dt_groupnorm_workspace_bytes(N, C, HW, G);
            void* ws = nullptr;
            int rc = backend_scratch(be, ws_bytes, &ws);
            if (rc) return rc;
            g_kernels += 2;
            return dt_groupnorm_silu(x->data, N, C, HW, G, p.in[1] ? (const float*)p.in[1]->data : nullptr,
                                     p.in[2] ? (const float*)p.in[2]->data : nullptr, p.eps, p.silu,
                                     root->data, ws, ws_bytes, root->type, st);
        }
        case K_QK: {
            const int es = elem_size(root->type);
            const int n_axes = (int)p.pos.size();
            for (const QkSeg& s : p.segs) {
                RopeAxisPos ap{};
                for (int a = 0; a < n_axes; ++a) {
                    ap.stride[a] = p.pos[a]->nb[0] / 4;
                    ap.ptr[a] = (const int32_t*)p.pos[a]->data + s.tok0 * ap.stride[a];
                }
                const dt_tensor* q = s.q;
                char* out = (char*)root->data + s.tok0 * root->nb[2];
                ++g_kernels;
                int rc = qk_launch(q->data, nullptr, out, nullptr, (const float*)s.w->data, nullptr,
                                   s.tokens, q->ne[1], q->ne[0], q->nb[2] / es, q->nb[1] / es,
                                   root->nb[2] / es, root->nb[1] / es, s.eps, ap,
                                   n_axes, p.axis_dim, p.base, nullptr, 0, root->type, st);
                if (rc) return rc;
            }
            return DT_OK;
        }
        case K_SILU:
            ++g_kernels;
            return dt_op_unary(DT_UN_SILU, p.in[0], root, 0.f, 0.f, st);
        case K_GEMM_ADD:
            ++g_kernels;
            return run_mul_mat(be, p.in[0], root, p.in[1]);
        case K_GEMM_GROUP:
            ++g_kernels;
            return run_gemm_group(be, p.members);
        case K_QK_SWIGLU: {
            const int es = elem_size(root->type);
            const int n_axes = (int)p.pos.size();
            RopeAxisPos ap{};
            for (int a = 0; a < n_axes; ++a) {
                ap.stride[a] = p.pos[a]->nb[0] / 4;
                ap.ptr[a] = (const int32_t*)data_of(p.pos[a]);
            }
            const QkSeg& qs = p.segs[0];
            const dt_tensor* q = qs.q;
            int64_t rows, gs, us, ys;
            row_layout(p.sw[0], &rows, &gs);
            row_layout(p.sw[1], &rows, &us);
            row_layout(p.sw[2], &rows, &ys);
            ++g_kernels;
            const bool two = p.kroot != nullptr;  // else the root alone (its block's q is in the attention)
            return qk_swiglu_launch(data_of(q), two ? data_of(p.kseg.q) : nullptr, root->data,
                                    two ? p.kroot->data : nullptr, (const float*)data_of(qs.w),
                                    two ? (const float*)data_of(p.kseg.w) : nullptr, qs.tokens,
                                    q->ne[1], q->ne[0], q->nb[2] / es, q->nb[1] / es, root->nb[2] / es,
                                    root->nb[1] / es, qs.eps, ap, n_axes, p.axis_dim, p.base, nullptr, 0,
                                    data_of(p.sw[0]), gs, data_of(p.sw[1]), us, p.sw[2]->data, ys, rows,
                                    p.sw[2]->ne[0], root->type, st);
        }
        case K_RES_ADALN: {
            int64_t rows, hs, os, rs, ys;
            row_layout(p.in[0], &rows, &hs);
            row_layout(p.in[1], &rows, &os);
            row_layout(p.in[3], &rows, &rs);
            row_layout(root, &rows, &ys);
            ++g_kernels;
            return residual_adaln_launch(data_of(p.in[0]), hs, data_of(p.in[1]), os, (const float*)data_of(p.in[2]),
                                         p.in[3]->data, rs, (const float*)data_of(p.in[5]),
                                         (const float*)data_of(p.in[4]), p.addend, root->data, ys, rows, root->ne[0],
                                         p.eps, root->type, st);
        }
        case K_CONV:
            return run_conv(be, root, p.in[0], p.in[1], p.in[2], p.in[3], p.up2, &p);
        case K_ATTN_QK:
            ++g_kernels;
            return run_attn_qk(be, root, p);
        case K_DEFERRED:
            return DT_OK;  // ran in its group's launch
        default:
            return fail(DT_ERR_INVALID_ARG, "run_plan: no plan");
    }
}

int run_unfused(dt_backend* be, dt_tensor* t) {
    hipStream_t st = backend_stream(be);
    switch (t->op) {
        case DT_OP_NONE:
            return DT_OK;
        case DT_OP_VIEW:
            DT_REQUIRE(t->src[0] && t->src[0]->data, "dt_graph_compute: VIEW of a node without data");
            t->data = (char*)t->src[0]->data + view_offset(t);
            return DT_OK;
        case DT_OP_UNARY:
            ++g_kernels;
            return dt_op_unary(t->op_params[0], t->src[0], t, fparam(t, 1), fparam(t, 2), st);
        case DT_OP_ADD:
        case DT_OP_SUB:
        case DT_OP_MUL:
        case DT_OP_DIV:
            ++g_kernels;
            return dt_op_binary(t->op - DT_OP_ADD, t->src[0], t->src[1], t, st);
        case DT_OP_SCALE:
            ++g_kernels;
            return dt_op_unary(DT_UN_SCALE, t->src[0], t, fparam(t, 0), 0.f, st);
        case DT_OP_SIGMOID:
            ++g_kernels;
            return dt_op_unary(DT_UN_SIGMOID, t->src[0], t, 0.f, 0.f, st);
        case DT_OP_FILL:
            ++g_kernels;
            return dt_op_unary(DT_UN_FILL, nullptr, t, fparam(t, 0), 0.f, st);
        case DT_OP_NORM:
            ++g_kernels;
            return dt_op_norm(t->src[0], t, fparam(t, 0), st);
        case DT_OP_RMS_NORM:
            ++g_kernels;
            return dt_op_rms_norm(t->src[0], t, fparam(t, 0), st);
        case DT_OP_ROPE: {
            const dt_tensor* ps = t->src[1];
            DT_REQUIRE(ps && ps->type == DT_TYPE_I32 && ps->nb[0] == 4,
                       "dt_graph_compute: ROPE positions must be contiguous I32");
            ++g_kernels;
            return dt_op_rope_ext(t->src[0], (const int32_t*)ps->data, t, t->op_params[0],
                                  t->op_params[1], fparam(t, 2), fparam(t, 3), fparam(t, 4),
                                  fparam(t, 5), st);
        }
        case DT_OP_CONCAT:
            ++g_kernels;
            return dt_op_concat(t->src[0], t->src[1], t->op_params[0], t, st);
        case DT_OP_CPY:
            ++g_kernels;
            return dt_op_cpy(t->src[0], t, st);
        case DT_OP_MUL_MAT:
            ++g_kernels;
            return run_mul_mat(be, t, t, nullptr);
        case DT_OP_FLASH_ATTN_EXT:
            ++g_kernels;
            if (t->src[0] && t->src[0]->type == DT_TYPE_F32 && t->src[1] && t->src[2] && !t->src[3])
                return run_flash_attn_f32(be, t);
            return run_flash_attn(st, t);
        case DT_OP_CONV_2D_DIRECT:
            DT_REQUIRE(t->src[0] && t->src[1], "dt_graph_compute: CONV_2D_DIRECT needs a weight and an input");
            return run_conv(be, t, t->src[1], t->src[0], nullptr, t, 0);
        case DT_OP_UPSCALE:
            ++g_kernels;
            return run_upscale(st, t);
        default:
            return fail(DT_ERR_UNSUPPORTED, "dt_graph_compute: op %d not supported", t->op);
    }
}

}  // namespace
}  // namespace dit

namespace dit {
namespace {

// ---- memory hazards of a plan under the caller's allocation -------------------
//
// A fused launch reads its external inputs at its own position and writes
// every output it keeps there.  Some launches move work relative to node
// order: a chain reads its first node's inputs at its last node, residual +
// adaLN writes r later, grouped GEMMs and QK+SwiGLU write later nodes'
// outputs earlier, an attention reads q's pre-norm input at the attention.
// An allocator that follows only node order (ggml_gallocr, Context.hpp:118-135)
// may hand an input's memory to another node after the input's last reader
// in node order, or give a later node's output memory that is still live
// earlier.  check_plan_memory replays the plan's launches in execution order
// over the nodes' actual address ranges and reports every launch that would
// read memory another node has overwritten (or that another launch overwrote
// too early); plan_checked then keeps those launches from moving work, and
// as a last step from fusing, until the replay is clean.

struct Span {
    uintptr_t lo = 0, hi = 0;
};

// Bytes a tensor's elements span from its data address (views resolved).
bool span_of(const dt_tensor* t, Span* s) {
    const void* d = data_of(t);
    if (!d) return false;
    for (int i = 0; i < 4; ++i)
        if (t->ne[i] <= 0) return false;
    int64_t ext = 0;
    if (t->type == DT_TYPE_Q8_0_SPLIT) {
        ext = (int64_t)dt_q8_0_split_bytes(t->ne[1], t->ne[0]);
    } else if (t->type == DT_TYPE_CONV2D_PACKED) {
        ext = (int64_t)dt_conv2d_packed_bytes(t->ne[3], t->ne[2], t->ne[0]);
    } else {
        const int es = elem_size(t->type);
        int d0 = 1;
        if (es) {
            ext = es;
        } else if (t->type == DT_TYPE_Q8_0 || t->type == DT_TYPE_Q4_K) {
            const int64_t blk = t->type == DT_TYPE_Q8_0 ? 32 : 256, bb = t->type == DT_TYPE_Q8_0 ? 34 : 144;
            ext = (t->ne[0] + blk - 1) / blk * bb;
        } else {
            return false;
        }
        if (es) d0 = 0;
        for (int i = d0; i < 4; ++i) ext += (t->ne[i] - 1) * (int64_t)t->nb[i];
    }
    s->lo = (uintptr_t)d;
    s->hi = s->lo + (uintptr_t)ext;
    return s->hi > s->lo;
}

// Which tensor's value lives at each address: disjoint [lo, hi) segments.
class OwnerMap {
public:
    struct Seg {
        uintptr_t hi;
        int owner;   // value identity (a node index, or kLeaf)
        int writer;  // node whose launch wrote it
    };
    void write(const Span& s, int owner, int writer) {
        auto it = m_.lower_bound(s.lo);
        if (it != m_.begin()) {
            auto pv = std::prev(it);
            if (pv->second.hi > s.lo) {
                const Seg tail = pv->second;
                pv->second.hi = s.lo;
                if (tail.hi > s.hi) m_[s.hi] = tail;
            }
        }
        it = m_.lower_bound(s.lo);
        while (it != m_.end() && it->first < s.hi) {
            const Seg seg = it->second;
            it = m_.erase(it);
            if (seg.hi > s.hi) {
                m_[s.hi] = seg;
                break;
            }
        }
        m_[s.lo] = Seg{s.hi, owner, writer};
    }
    // A segment inside s holding another value than `owner` (bytes nobody
    // wrote are taken as intact), or nullptr.
    const Seg* foreign(const Span& s, int owner) const {
        auto it = m_.upper_bound(s.lo);
        if (it != m_.begin()) --it;
        for (; it != m_.end() && it->first < s.hi; ++it)
            if (it->second.hi > s.lo && it->second.owner != owner) return &it->second;
        return nullptr;
    }

private:
    std::map<uintptr_t, Seg> m_;
};

constexpr int kLeaf = -2;

// Value identity of the memory t reads: its storage root (VIEW chains
// resolved), a node index or kLeaf for tensors outside the list.
int value_of(const Graph& g, const dt_tensor* t) {
    while (t && t->op == DT_OP_VIEW) t = t->src[0];
    if (!t) return kLeaf;
    auto it = g.index.find(t);
    return it == g.index.end() ? kLeaf : it->second;
}

bool launch_moves(const Plan& p) {
    return p.kind == K_RES_ADALN || p.kind == K_ATTN_QK || p.kind == K_GEMM_GROUP || p.kind == K_QK_SWIGLU;
}

// Launches (by position) that read clobbered memory or clobber live memory.
void check_plan_memory(const Graph& g, dt_tensor** nodes, int n, const std::vector<Plan>& plans,
                       std::vector<int>& blamed) {
    std::vector<std::vector<int>> members(n);
    for (int j = 0; j < n; ++j) members[g.runs_at[j]].push_back(j);
    std::vector<char> is_blamed(n, 0);
    auto blame = [&](int pos) {
        if (pos >= 0 && pos < n && !is_blamed[pos]) {
            is_blamed[pos] = 1;
            blamed.push_back(pos);
        }
    };
    // A CPY into a destination writes on behalf of the destination's value.
    auto write_identity = [&](int j) {
        const dt_tensor* t = nodes[j];
        return t->op == DT_OP_CPY && t->src[1] ? value_of(g, t->src[1]) : j;
    };
    OwnerMap owners;
    std::vector<std::pair<Span, int>> reads, writes;
    for (int p = 0; p < n; ++p) {
        if (g.claimed[p] || plans[p].kind == K_DEFERRED) continue;  // not a launch position
        reads.clear();
        writes.clear();
        const bool fused = plans[p].kind != K_NONE;
        for (int j : members[p]) {
            const dt_tensor* t = nodes[j];
            for (int k = 0; k < 4; ++k) {
                const dt_tensor* s = t->src[k];
                if (!s) continue;
                auto si = g.index.find(s);
                if (si != g.index.end() && g.runs_at[si->second] == p) continue;  // produced in this launch
                Span sp;
                if (!span_of(s, &sp)) continue;
                const int want = value_of(g, s);
                if (const OwnerMap::Seg* f = owners.foreign(sp, want)) {
                    bool found = false;
                    if (j < p) {  // the read moved later than its node
                        blame(p);
                        found = true;
                    }
                    if (g.runs_at[f->writer] < f->writer) {  // the overwrite moved earlier
                        blame(g.runs_at[f->writer]);
                        found = true;
                    }
                    if (want >= 0 && g.runs_at[want] < want) {  // the value was written early, then reused
                        blame(g.runs_at[want]);
                        found = true;
                    }
                    (void)found;  // nothing moved: the node order itself reads it so
                }
                reads.push_back({sp, want});
            }
        }
        for (int j : members[p]) {
            const dt_tensor* t = nodes[j];
            if (g.claimed[j] || t->op == DT_OP_VIEW || t->op == DT_OP_NONE) continue;
            Span sp;
            if (span_of(t, &sp)) writes.push_back({sp, j});
        }
        // A fused kernel may write over an input only element for element;
        // a conv only over its residual, and only while its input is
        // elsewhere.
        const Plan& pl = plans[p];
        Span rs{}, xs{};
        const bool conv_res = pl.kind == K_CONV && pl.in[4] && span_of(pl.in[4], &rs) && span_of(pl.in[0], &xs);
        if (fused)
            for (const auto& w : writes)
                for (const auto& r : reads) {
                    const bool overlap = w.first.lo < r.first.hi && r.first.lo < w.first.hi;
                    const bool same = w.first.lo == r.first.lo && w.first.hi == r.first.hi;
                    const bool res_in_place = conv_res && same && r.first.lo == rs.lo && r.first.hi == rs.hi &&
                                              !(w.first.lo < xs.hi && xs.lo < w.first.hi);
                    if (overlap && (!same || pl.kind == K_ATTN_QK || pl.kind == K_GEMM_GROUP ||
                                    (pl.kind == K_CONV && !res_in_place)))
                        blame(p);
                }
        for (const auto& w : writes) owners.write(w.first, write_identity(w.second), w.second);
    }
}

int plan_graph(dt_tensor** nodes, int32_t n_nodes, Graph& g, std::vector<Plan>& plans);

// The fusion plan, then (check) the memory replay, repeated with the blamed
// launches held at their positions (then unfused) until it is clean.
int plan_checked(dt_tensor** nodes, int32_t n, Graph& g, std::vector<Plan>& plans, bool check, int* kept_apart) {
    std::vector<char> nomove(n, 0), banned(n, 0);
    if (kept_apart) *kept_apart = 0;
    for (;;) {
        g = Graph();
        g.nomove = nomove;
        g.banned = banned;
        int rc = plan_graph(nodes, n, g, plans);
        if (rc || !check) return rc;
        std::vector<int> blamed;
        check_plan_memory(g, nodes, n, plans, blamed);
        bool changed = false;
        for (int p : blamed) {
            if (!nomove[p] && launch_moves(plans[p])) {
                nomove[p] = 1;
            } else if (!banned[p] && plans[p].kind != K_NONE) {
                banned[p] = nomove[p] = 1;
            } else {
                continue;
            }
            changed = true;
            if (kept_apart) ++*kept_apart;
        }
        if (!changed) return DT_OK;
    }
}

int plan_graph(dt_tensor** nodes, int32_t n_nodes, Graph& g, std::vector<Plan>& plans) {
    g.nodes = nodes;
    if ((int)g.nomove.size() != n_nodes) g.nomove.assign(n_nodes, 0);
    if ((int)g.banned.size() != n_nodes) g.banned.assign(n_nodes, 0);
    g.claimed.assign(n_nodes, 0);
    g.deferred.assign(n_nodes, 0);
    g.root.assign(n_nodes, -1);
    g.runs_at.resize(n_nodes);
    for (int i = 0; i < n_nodes; ++i) g.runs_at[i] = i;
    for (int i = 0; i < n_nodes; ++i) {
        DT_REQUIRE(nodes[i] != nullptr, "dt_graph: node %d is null", i);
        g.index[nodes[i]] = i;
        for (int s = 0; s < 4; ++s)
            if (nodes[i]->src[s]) {
                g.uses[nodes[i]->src[s]]++;
                g.consumers[nodes[i]->src[s]].push_back(i);
            }
    }
    plans.assign(n_nodes, Plan());
    for (int i = n_nodes - 1; i >= 0; --i) {
        if (g.claimed[i] || g.deferred[i] || g.banned[i]) continue;
        dt_tensor* t = nodes[i];
        Plan& p = plans[i];
        g.current_root = i;
        if (match_attn_qk(g, t, p) || match_qk(g, t, p) || match_groupnorm(g, t, p) || match_res_adaln(g, t, p) ||
            match_adaln(g, t, p) ||
            match_swiglu(g, t, p) || match_gated(g, t, p) || match_silu(g, t, p) ||
            match_gemm_add(g, t, p) || match_conv_residual(g, t, p) || match_conv(g, t, p))
            continue;
        p = Plan();
    }
    for (int i = 0; i < n_nodes; ++i) {
        if (g.claimed[i]) g.runs_at[i] = g.root[i];
        if (g.deferred[i]) plans[i].kind = K_DEFERRED;
    }
    group_gemms(g, nodes, n_nodes, plans);
    merge_qk_swiglu(g, nodes, n_nodes, plans);
    defer_gemms(g, nodes, n_nodes, plans);
    return DT_OK;
}

}  // namespace
}  // namespace dit

extern "C" int dt_graph_plan_ex(dt_tensor** nodes, int32_t n_nodes, int32_t* fused_into, int32_t* runs_at) {
    using namespace dit;
    DT_REQUIRE(n_nodes >= 0 && (nodes || n_nodes == 0) && (fused_into || n_nodes == 0),
               "dt_graph_plan: bad arguments");
    Graph g;
    std::vector<Plan> plans;
    int rc = plan_checked(nodes, n_nodes, g, plans, false, nullptr);
    if (rc) return rc;
    for (int i = 0; i < n_nodes; ++i) {
        fused_into[i] = g.claimed[i] ? g.root[i] : -1;
        if (runs_at) runs_at[i] = g.runs_at[i];
    }
    return DT_OK;
}

extern "C" int dt_graph_plan(dt_tensor** nodes, int32_t n_nodes, int32_t* fused_into) {
    return dt_graph_plan_ex(nodes, n_nodes, fused_into, nullptr);
}

extern "C" int dt_graph_plan_checked(dt_tensor** nodes, int32_t n_nodes, int32_t* fused_into, int32_t* runs_at,
                                     int32_t* launches_held) {
    using namespace dit;
    DT_REQUIRE(n_nodes >= 0 && (nodes || n_nodes == 0) && (fused_into || n_nodes == 0),
               "dt_graph_plan_checked: bad arguments");
    Graph g;
    std::vector<Plan> plans;
    int held = 0;
    int rc = plan_checked(nodes, n_nodes, g, plans, true, &held);
    if (rc) return rc;
    for (int i = 0; i < n_nodes; ++i) {
        fused_into[i] = g.claimed[i] ? g.root[i] : -1;
        if (runs_at) runs_at[i] = g.runs_at[i];
    }
    if (launches_held) *launches_held = held;
    return DT_OK;
}

namespace dit {
namespace {
thread_local int g_held = 0;
}  // namespace
}  // namespace dit

extern "C" int dt_graph_compute_ex(dt_backend* be, dt_tensor** nodes, int32_t n_nodes, uint32_t flags) {
    using namespace dit;
    DT_REQUIRE(be != nullptr, "dt_graph_compute: null backend");
    DT_REQUIRE(n_nodes >= 0 && (nodes || n_nodes == 0), "dt_graph_compute: bad node list");
    DT_REQUIRE((flags & ~(uint32_t)DT_GRAPH_ALLOC_RUNS_AT) == 0, "dt_graph_compute: unknown flags 0x%x", flags);
    g_kernels = 0;
    g_fused = 0;
    g_held = 0;
    Graph g;
    std::vector<Plan> plans;
    int rc = plan_checked(nodes, n_nodes, g, plans, !(flags & DT_GRAPH_ALLOC_RUNS_AT), &g_held);
    if (rc) return rc;
    for (int i = 0; i < n_nodes; ++i) {
        if (g.claimed[i]) {
            ++g_fused;
            continue;
        }
        rc = plans[i].kind != K_NONE ? run_plan(be, nodes[i], plans[i]) : run_unfused(be, nodes[i]);
        if (rc) return rc;
    }
    return DT_OK;
}

extern "C" int dt_graph_compute(dt_backend* be, dt_tensor** nodes, int32_t n_nodes) {
    return dt_graph_compute_ex(be, nodes, n_nodes, 0);
}

extern "C" int dt_graph_last_stats(int32_t* kernels_launched, int32_t* nodes_fused) {
    if (kernels_launched) *kernels_launched = dit::g_kernels;
    if (nodes_fused) *nodes_fused = dit::g_fused;
    return DT_OK;
}

extern "C" int dt_graph_last_stats_ex(int32_t* kernels_launched, int32_t* nodes_fused, int32_t* launches_held) {
    dt_graph_last_stats(kernels_launched, nodes_fused);
    if (launches_held) *launches_held = dit::g_held;
    return DT_OK;
}
