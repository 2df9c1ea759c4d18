// modules.hpp -- the reference's nn / Flux2 module call sites for the DiT
// elementwise chain, restated on the host Tensor layer so that they record
// the same node graph the reference records through its Runtime:
//   LayerNorm      src/nn/modules/normalization/LayerNorm.cpp:16-32
//   RMSNorm        src/nn/modules/normalization/RMSNorm.cpp:12-22
//   GroupNorm      src/nn/modules/normalization/GroupNorm.cpp:25-108
//   SiLU           src/nn/SiLU.hpp:9-13
//   Conv2d         src/nn/modules/conv/Conv2d.cpp:5-102
//   Upsample2D     src/diffusers/models/resnet/Upsample2D.cpp:6-73
//   Flux2PosEmbed  src/diffusers/models/transformers/flux2/Flux2PosEmbed.hpp:18-109
//   Flux2SwiGLU    src/diffusers/models/transformers/flux2/Flux2SwiGLU.hpp:17-21
//   Flux2Modulation::split  Flux2Modulation.hpp:24-41
// plus the modulation / residual expressions of the transformer blocks
// (Flux2SingleTransformerBlock.hpp:50-58, Flux2TransformerBlock.hpp:63-111).
// Parameters are F32 leaves created at construction (a RuntimeScope must be
// active); callers bind their data through HipRuntime::bind.
#pragma once

#include <array>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "tensor.hpp"

namespace dit {
namespace host {

inline Tensor parameter(const Tensor::Shape& shape, int32_t type = DT_TYPE_F32) {
    Tensor p = Tensor::empty(shape, type);
    current_runtime().set_param(*p);
    return p;
}

// The module tree of src/nn/Module.hpp: named children and parameters, so
// every parameter has the dotted path the reference's loaders use
// ("transformer_blocks.0.attn.to_q.weight").  Members are held by value and
// registered by address, so modules are neither copied nor moved.
class Module {
public:
    Module() = default;
    Module(const Module&) = delete;
    Module& operator=(const Module&) = delete;
    virtual ~Module() = default;

    void named_parameters(std::vector<std::pair<std::string, Tensor>>& out,
                          const std::string& prefix = "") const {
        for (const auto& p : params_) out.emplace_back(prefix + p.first, *p.second);
        for (const auto& c : children_) c.second->named_parameters(out, prefix + c.first + ".");
    }

protected:
    void register_parameter(const std::string& name, Tensor& t) { params_.emplace_back(name, &t); }
    void register_module(const std::string& name, Module& m) { children_.emplace_back(name, &m); }

private:
    std::vector<std::pair<std::string, Tensor*>> params_;
    std::vector<std::pair<std::string, Module*>> children_;
};

class LayerNorm : public Module {
public:
    explicit LayerNorm(int64_t dim, float eps = 1e-5f, bool elementwise_affine = true, bool bias = true)
        : eps_(eps), affine_(elementwise_affine), bias_(bias) {
        if (affine_) {
            weight = parameter({dim});
            register_parameter("weight", weight);
            if (bias_) {
                this->bias = parameter({dim});
                register_parameter("bias", this->bias);
            }
        }
    }
    Tensor forward(Tensor x) const {
        x = Tensor(current_runtime().norm(*x, eps_), x.shape());
        if (affine_) {
            x = x * weight;
            if (bias_) x = x + bias;
        }
        return x;
    }
    Tensor weight, bias;

private:
    float eps_;
    bool affine_, bias_;
};

class RMSNorm : public Module {
public:
    explicit RMSNorm(int64_t dim, float eps = 1e-5f, bool elementwise_affine = true)
        : eps_(eps), affine_(elementwise_affine) {
        if (affine_) {
            weight = parameter({dim});
            register_parameter("weight", weight);
        }
    }
    Tensor forward(Tensor x) const {
        x = Tensor(current_runtime().rms_norm(*x, eps_), x.shape());
        if (affine_) x = x * weight;
        return x;
    }
    Tensor weight;

private:
    float eps_;
    bool affine_;
};

class GroupNorm : public Module {
public:
    GroupNorm(int64_t num_groups, int64_t num_channels, float eps = 1e-5f, bool affine = true,
              bool bias = true)
        : groups_(num_groups), eps_(eps), affine_(affine), bias_(bias) {
        if (affine_) {
            weight = parameter({num_channels});
            register_parameter("weight", weight);
            if (bias_) {
                this->bias = parameter({num_channels});
                register_parameter("bias", this->bias);
            }
        }
    }
    Tensor forward(Tensor input) const {
        const auto s = input.shape();
        const int64_t n = s[0], c = s[1], h = s[2], w = s[3];
        input = input.reshape({n, groups_, -1});
        input = Tensor(current_runtime().norm(*input, eps_), input.shape());
        input = input.reshape({n, c, h, w});
        if (affine_) {
            input = input * weight.reshape({1, c, 1, 1});
            if (bias_) input = input + bias.reshape({1, c, 1, 1});
        }
        return input;
    }
    Tensor weight, bias;

private:
    int64_t groups_;
    float eps_;
    bool affine_, bias_;
};

struct SiLU {
    // x * sigmoid(x): the composite the reference emits instead of ggml_silu.
    Tensor forward(const Tensor& x) const { return x * x.sigmoid(); }
};

inline int32_t& conv_weight_type_slot() {
    thread_local int32_t t = DT_TYPE_F32;
    return t;
}

// Scoped choice of the type new Conv2d weights are created with: F32 (the
// reference's parameters) or DT_TYPE_CONV2D_PACKED, a weight the loader packs
// once (dt_conv2d_pack_weights) so the executor does not repack it per call.
class ConvWeightType {
public:
    explicit ConvWeightType(int32_t type) : prev_(conv_weight_type_slot()) { conv_weight_type_slot() = type; }
    ~ConvWeightType() { conv_weight_type_slot() = prev_; }

private:
    int32_t prev_;
};

// Conv2d (src/nn/modules/conv/Conv2d.cpp:5-102): weight [Co, Ci, K, K] and
// bias [Co]; forward = conv_2d_direct on the contiguous input, then the bias
// broadcast as [1, Co, 1, 1].  The executor runs the pair as one convolution
// with the bias in its epilogue.
class Conv2d : public Module {
public:
    Conv2d(int64_t in_channels, int64_t out_channels, int64_t kernel_size, int64_t stride = 1, int64_t padding = 0,
           bool bias = true)
        : stride_(stride), padding_(padding), bias_(bias) {
        weight = parameter({out_channels, in_channels, kernel_size, kernel_size}, conv_weight_type_slot());
        register_parameter("weight", weight);
        if (bias_) {
            this->bias = parameter({out_channels});
            register_parameter("bias", this->bias);
        }
    }
    Tensor forward(Tensor x) const {
        if (!x.is_contiguous()) x = x.contiguous();
        const Tensor::Shape& ws = weight.shape();
        Tensor::Shape shape = x.shape();
        Node* y = current_runtime().conv_2d_direct(*weight, *x, (int)stride_, (int)stride_, (int)padding_,
                                                   (int)padding_, 1, 1);
        shape[1] = ws[0];
        shape[2] = (shape[2] + 2 * padding_ - ws[2]) / stride_ + 1;
        shape[3] = (shape[3] + 2 * padding_ - ws[3]) / stride_ + 1;
        Tensor out(y, shape);
        if (bias_) out = out + bias.reshape({1, ws[0], 1, 1});
        return out;
    }
    Tensor weight, bias;

private:
    int64_t stride_, padding_;
    bool bias_;
};

// Upsample2D (src/diffusers/models/resnet/Upsample2D.cpp:6-73): nearest 2x
// upscale, then an optional 3x3 conv (padding 1).  With the conv, the
// executor folds the upscale into the conv's input addressing.
class Upsample2D : public Module {
public:
    explicit Upsample2D(int64_t channels, bool use_conv = false, int64_t out_channels = -1) {
        if (use_conv) {
            conv_.reset(new Conv2d(channels, out_channels > 0 ? out_channels : channels, 3, 1, 1));
            register_module("conv", *conv_);
        }
    }
    Tensor forward(const Tensor& hidden_states) const {
        const Tensor::Shape& s = hidden_states.shape();
        Tensor h(current_runtime().upscale(*hidden_states, 2, ScaleMode::Nearest), {s[0], s[1], s[2] * 2, s[3] * 2});
        return conv_ ? conv_->forward(h) : h;
    }
    Conv2d* conv() const { return conv_.get(); }

private:
    std::unique_ptr<Conv2d> conv_;
};

class Flux2PosEmbed {
public:
    Flux2PosEmbed(int64_t theta, std::vector<int64_t> axes_dim) : theta_(theta), axes_(std::move(axes_dim)) {}

    // x: [..., head_dim]; position_ids: I32 [sequence, n_axes].  The per-axis
    // position columns (a narrow + squeeze, i.e. a CONT copy) are made once
    // per position tensor and shared by every later call on it, where the
    // reference re-derives them for q and k of every block.
    Tensor forward(const Tensor& x, const Tensor& position_ids) const {
        const std::vector<Tensor>& pos = columns(position_ids);
        std::vector<Tensor> sections;
        int64_t offset = 0;
        for (size_t axis = 0; axis < axes_.size(); ++axis) {
            const int64_t d = axes_[axis];
            Tensor x_axis = x.narrow(-1, offset, d);
            const Tensor& pos_axis = pos[axis];
            Node* r = current_runtime().rope_ext(*x_axis, *pos_axis, nullptr, (int)d, 0, 0,
                                                 (float)theta_, 1.0f, 0.0f, 1.0f, 0.0f, 0.0f);
            sections.emplace_back(r, x_axis.shape());
            offset += d;
        }
        return Tensor::cat(sections, -1);
    }

private:
    const std::vector<Tensor>& columns(const Tensor& position_ids) const {
        for (const auto& c : cache_)
            if (c.first == *position_ids) return c.second;
        std::vector<Tensor> cols;
        for (size_t axis = 0; axis < axes_.size(); ++axis) {
            Tensor p = position_ids.select(1, (int64_t)axis);  // narrow + squeeze (-> CONT)
            if (p.ndim() != 1) p = p.flatten(0, p.ndim() - 1);
            cols.push_back(p);
        }
        cache_.emplace_back(*position_ids, std::move(cols));
        return cache_.back().second;
    }

    int64_t theta_;
    std::vector<int64_t> axes_;
    mutable std::vector<std::pair<Node*, std::vector<Tensor>>> cache_;
};

struct Flux2SwiGLU {
    Tensor forward(const Tensor& gate, const Tensor& up) const { return SiLU().forward(gate) * up; }
};

struct Flux2Modulation {
    // [1, 3*sets*D] or [1, 1, 3*sets*D] -> per set {shift, scale, gate} views.
    static std::vector<std::array<Tensor, 3>> split(Tensor mod, int64_t sets) {
        if (mod.ndim() == 2) mod = mod.unsqueeze(1);
        auto parts = mod.chunk((int)(3 * sets), -1);
        std::vector<std::array<Tensor, 3>> out;
        for (int64_t i = 0; i < sets; ++i) out.push_back({parts[3 * i], parts[3 * i + 1], parts[3 * i + 2]});
        return out;
    }
};

// `(1.0f + scale) * norm(x) + shift` (Flux2SingleTransformerBlock.hpp:53).
inline Tensor adaln_modulate(const LayerNorm& norm, const Tensor& x, const Tensor& shift,
                             const Tensor& scale) {
    return (1.0f + scale) * norm.forward(x) + shift;
}

// `hidden + gate * out` (Flux2SingleTransformerBlock.hpp:58).
inline Tensor gated_residual(const Tensor& hidden, const Tensor& gate, const Tensor& out) {
    return hidden + gate * out;
}

}  // namespace host
}  // namespace dit
