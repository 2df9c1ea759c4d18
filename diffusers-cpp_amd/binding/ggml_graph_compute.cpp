// ggml_graph_compute.cpp -- reference-side translation of a ggml_cgraph into
// dt_tensor nodes for dt_graph_compute: the function a diffusers-cpp
// maintainer adds beside src/ggml/ExecutionRuntime.cpp and calls at its two
// ggml_backend_graph_compute sites (ExecutionRuntime.cpp:227, 254).
//
// Not built in this repository: it includes ggml.h, and ggml is an
// un-vendored submodule of the reference (.gitmodules:1-3).  Enum and field
// names follow public ggml; op-parameter slots are listed per op in
// ggml_op_map.tsv (next to this file), which tests/test_binding_map.py checks
// against this file and against the op set of a recorded Flux2 step.
//
// Memory: the reference allocates node memory with ggml_gallocr in node
// order (Context.hpp:118-135).  dt_graph_compute (flags 0) replays its
// fusion plan over those addresses and keeps any launch that would read
// memory gallocr has handed on at its own position, or unfused.
#include <cstring>
#include <unordered_map>
#include <vector>

#include "dit_hip.h"
#include "ggml.h"

namespace {

// dt op of a ggml node, or -1 for an op this backend does not run (the
// caller then keeps the graph on ggml).
int32_t dt_op_of(const ggml_tensor* t) {
    switch (t->op) {
        case GGML_OP_NONE:           return DT_OP_NONE;
        case GGML_OP_ADD:            return DT_OP_ADD;
        case GGML_OP_SUB:            return DT_OP_SUB;
        case GGML_OP_MUL:            return DT_OP_MUL;
        case GGML_OP_DIV:            return DT_OP_DIV;
        case GGML_OP_SCALE:          return DT_OP_SCALE;
        case GGML_OP_FILL:           return DT_OP_FILL;
        case GGML_OP_NORM:           return DT_OP_NORM;
        case GGML_OP_RMS_NORM:       return DT_OP_RMS_NORM;
        case GGML_OP_ROPE:           return DT_OP_ROPE;
        case GGML_OP_CONCAT:         return DT_OP_CONCAT;
        case GGML_OP_CPY:
        case GGML_OP_CONT:
        case GGML_OP_DUP:            return DT_OP_CPY;
        case GGML_OP_VIEW:
        case GGML_OP_RESHAPE:
        case GGML_OP_PERMUTE:
        case GGML_OP_TRANSPOSE:      return DT_OP_VIEW;
        case GGML_OP_MUL_MAT:        return DT_OP_MUL_MAT;
        case GGML_OP_FLASH_ATTN_EXT: return DT_OP_FLASH_ATTN_EXT;
        case GGML_OP_CONV_2D_DIRECT: return DT_OP_CONV_2D_DIRECT;
        case GGML_OP_UPSCALE:        return DT_OP_UPSCALE;
        case GGML_OP_SQRT:
        case GGML_OP_LOG:
        case GGML_OP_SIN:
        case GGML_OP_COS:
        case GGML_OP_CLAMP:          return DT_OP_UNARY;
        case GGML_OP_UNARY:
            switch (ggml_get_unary_op(t)) {
                case GGML_UNARY_OP_SIGMOID: return DT_OP_SIGMOID;
                case GGML_UNARY_OP_EXP:     return DT_OP_UNARY;
                default:                    return -1;
            }
        default:                     return -1;
    }
}

// DT_UN_* kind of a node dt_op_of maps to DT_OP_UNARY.
int32_t dt_unary_of(const ggml_tensor* t) {
    switch (t->op) {
        case GGML_OP_SQRT:  return DT_UN_SQRT;
        case GGML_OP_LOG:   return DT_UN_LOG;
        case GGML_OP_SIN:   return DT_UN_SIN;
        case GGML_OP_COS:   return DT_UN_COS;
        case GGML_OP_CLAMP: return DT_UN_CLAMP;
        case GGML_OP_UNARY:
            switch (ggml_get_unary_op(t)) {
                case GGML_UNARY_OP_EXP: return DT_UN_EXP;
                default:                return -1;
            }
        default:            return -1;
    }
}

float f32_param(const ggml_tensor* t, int i) {
    float f;
    std::memcpy(&f, &t->op_params[i], 4);
    return f;
}

}  // namespace

// Returns GGML_STATUS_SUCCESS, or GGML_STATUS_FAILED with dt_last_error()
// set by the library, or for a node this backend does not run.
ggml_status dt_compute_ggml_graph(dt_backend* be, ggml_cgraph* gf) {
    const int n = ggml_graph_n_nodes(gf);
    std::vector<dt_tensor> nodes(n);
    std::unordered_map<const ggml_tensor*, dt_tensor*> map;
    std::vector<dt_tensor> leaves;  // sources that are not graph nodes
    leaves.reserve(4 * (size_t)n + 1);
    auto lookup = [&](const ggml_tensor* s) -> dt_tensor* {
        if (!s) return nullptr;
        auto it = map.find(s);
        if (it != map.end()) return it->second;
        leaves.emplace_back();
        dt_tensor& d = leaves.back();
        std::memset(&d, 0, sizeof d);
        d.type = (int32_t)s->type;
        for (int i = 0; i < 4; ++i) {
            d.ne[i] = s->ne[i];
            d.nb[i] = (int64_t)s->nb[i];
        }
        d.data = s->data;
        d.op = DT_OP_NONE;
        return map[s] = &d;
    };
    for (int i = 0; i < n; ++i) map[ggml_graph_node(gf, i)] = &nodes[i];
    std::vector<dt_tensor*> order(n);
    for (int i = 0; i < n; ++i) {
        const ggml_tensor* t = ggml_graph_node(gf, i);
        dt_tensor& d = nodes[i];
        std::memset(&d, 0, sizeof d);
        d.op = dt_op_of(t);
        if (d.op < 0) return GGML_STATUS_FAILED;
        d.type = (int32_t)t->type;
        for (int k = 0; k < 4; ++k) {
            d.ne[k] = t->ne[k];
            d.nb[k] = (int64_t)t->nb[k];
        }
        d.data = t->data;
        d.flags = (t->flags & GGML_TENSOR_FLAG_OUTPUT) ? DT_FLAG_OUTPUT : 0;
        for (int k = 0; k < 4; ++k) d.src[k] = lookup(t->src[k]);
        switch (d.op) {
            case DT_OP_VIEW: {  // view_src + view_offs
                d.src[0] = lookup(t->view_src);
                const uint64_t off = t->view_offs;
                d.op_params[0] = (int32_t)(uint32_t)off;
                d.op_params[1] = (int32_t)(off >> 32);
                break;
            }
            case DT_OP_ROPE:  // ggml: {n_past, n_dims, mode, n_ctx_orig, base@5, scale@6, ext@7, attn@8}
                d.op_params[0] = t->op_params[1];
                d.op_params[1] = t->op_params[2];
                std::memcpy(&d.op_params[2], &t->op_params[5], 4 * 4);
                break;
            case DT_OP_UNARY: {  // kind @0; clamp's min, max @1, @2
                const int32_t kind = dt_unary_of(t);
                if (kind < 0) return GGML_STATUS_FAILED;
                d.op_params[0] = kind;
                if (t->op == GGML_OP_CLAMP) {
                    d.op_params[1] = t->op_params[0];
                    d.op_params[2] = t->op_params[1];
                }
                break;
            }
            case DT_OP_SCALE:  // ggml_scale keeps {s, b}; this backend scales only
                if (f32_param(t, 1) != 0.0f) return GGML_STATUS_FAILED;
                d.op_params[0] = t->op_params[0];
                break;
            case DT_OP_UPSCALE:  // ggml keeps the mode @0; the factor is the ne ratio
                if ((t->op_params[0] & 0xFF) != GGML_SCALE_MODE_NEAREST || t->ne[0] % t->src[0]->ne[0] ||
                    t->ne[0] / t->src[0]->ne[0] != t->ne[1] / t->src[0]->ne[1])
                    return GGML_STATUS_FAILED;
                d.op_params[0] = (int32_t)(t->ne[0] / t->src[0]->ne[0]);
                break;
            default:  // FILL value, NORM / RMS_NORM eps, CONCAT dim, attention scale, conv s/p/d @0..
                std::memcpy(d.op_params, t->op_params, sizeof d.op_params);
                break;
        }
        order[i] = &d;
    }
    return dt_graph_compute(be, order.data(), n) == DT_OK ? GGML_STATUS_SUCCESS : GGML_STATUS_FAILED;
}
