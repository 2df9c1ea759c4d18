// resnet.hpp -- ResnetBlock2D (src/diffusers/models/resnet/ResnetBlock2D.hpp,
// ResnetBlock2D.inl:7-195), the residual block of the VAE decoder's mid and
// up blocks (UNetMidBlock2D.cpp:52, UpDecoderBlock2D.cpp:28), and
// UpDecoderBlock2D (src/diffusers/models/unets/unet2d/UpDecoderBlock2D.cpp:6-74),
// on the host Tensor layer.  ResnetBlock2D records the reference's node
// sequence:
//   norm1 -> SiLU -> conv1 [-> + time_emb_proj(SiLU(temb))[:, :, None, None]]
//   -> norm2 -> SiLU -> conv2, then (shortcut(x) + h) / output_scale_factor
// and the executor runs each GroupNorm + SiLU as one kernel and conv2 with
// the residual ADD and the SCALE in its epilogue.
#pragma once

#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

#include "flux2.hpp"

namespace dit {
namespace host {

template <class NonLinearity = SiLU>
class ResnetBlock2D : public Module {
public:
    // The reference constructor's arguments, in its order.  pre_norm must
    // be true and up / down false (the reference throws otherwise, as here);
    // conv_shortcut, dropout and skip_time_act do not change the inference
    // graph.
    explicit ResnetBlock2D(int64_t in_channels, std::optional<int64_t> out_channels = std::nullopt,
                           std::optional<int64_t> conv_shortcut = std::nullopt, float dropout = 0.0f,
                           std::optional<int64_t> temb_channels = 512, int64_t groups = 32,
                           std::optional<int64_t> groups_out = std::nullopt, bool pre_norm = true, float eps = 1e-6f,
                           bool skip_time_act = false, int64_t kernel_size = 3, float output_scale_factor = 1.0f,
                           std::optional<bool> use_in_shortcut = std::nullopt, bool up = false, bool down = false,
                           bool conv_shortcut_bias = true, std::optional<int64_t> conv_2d_out_channels = std::nullopt)
        : output_scale_factor_(output_scale_factor),
          norm1(groups, in_channels, eps),
          conv1(in_channels, out_channels.value_or(in_channels), kernel_size, 1, kernel_size / 2),
          norm2(groups_out.value_or(groups), out_channels.value_or(in_channels), eps),
          conv2(out_channels.value_or(in_channels), conv_2d_out_channels.value_or(out_channels.value_or(in_channels)),
                kernel_size, 1, kernel_size / 2) {
        (void)conv_shortcut;
        (void)dropout;
        (void)skip_time_act;
        if (!pre_norm) throw std::invalid_argument("ResnetBlock2D: 'pre_norm': not implemented");
        if (up) throw std::invalid_argument("ResnetBlock2D: 'up': not implemented");
        if (down) throw std::invalid_argument("ResnetBlock2D: 'down': not implemented");
        const int64_t out = out_channels.value_or(in_channels);
        const int64_t c2 = conv_2d_out_channels.value_or(out);
        register_module("norm1", norm1);
        register_module("conv1", conv1);
        if (temb_channels) {
            time_emb_proj_.reset(new Linear(*temb_channels, out));
            register_module("time_emb_proj", *time_emb_proj_);
        }
        register_module("norm2", norm2);
        register_module("conv2", conv2);
        if (use_in_shortcut.value_or(in_channels != c2)) {
            conv_shortcut_.reset(new Conv2d(in_channels, c2, 1, 1, 0, conv_shortcut_bias));
            register_module("conv_shortcut", *conv_shortcut_);
        }
    }

    // temb is used when the block has a time_emb_proj (ResnetBlock2D.inl:129).
    Tensor forward(const Tensor& input_tensor, const Tensor* temb = nullptr) const {
        const NonLinearity act;
        Tensor h = act.forward(norm1.forward(input_tensor));
        h = conv1.forward(h);
        if (time_emb_proj_ && temb) {
            Tensor t = time_emb_proj_->forward(act.forward(*temb));
            const Tensor::Shape& s = t.shape();
            h = h + t.reshape({s[0], s[1], 1, 1});
        }
        h = act.forward(norm2.forward(h));
        h = conv2.forward(h);
        const Tensor x = conv_shortcut_ ? conv_shortcut_->forward(input_tensor) : input_tensor;
        return (x + h) / output_scale_factor_;
    }

    Linear* time_emb_proj() const { return time_emb_proj_.get(); }
    Conv2d* conv_shortcut() const { return conv_shortcut_.get(); }

private:
    float output_scale_factor_;

public:
    GroupNorm norm1;
    Conv2d conv1;
    GroupNorm norm2;
    Conv2d conv2;

private:
    std::unique_ptr<Linear> time_emb_proj_;
    std::unique_ptr<Conv2d> conv_shortcut_;
};

// UpDecoderBlock2D (UpDecoderBlock2D.cpp:6-74): num_layers ResnetBlock2D
// (the first in_channels -> out_channels, the rest out -> out; groups
// resnet_groups, eps resnet_eps, no temb projection unless temb_channels),
// then with add_upsample an Upsample2D with its 3x3 conv.  As in the
// reference, forward does not pass temb to the resnets.  Parameters are
// named resnets.<i>.* and upsamplers.0.conv.*.
class UpDecoderBlock2D : public Module {
public:
    UpDecoderBlock2D(int64_t in_channels, int64_t out_channels, std::optional<int64_t> resolution_idx = std::nullopt,
                     float dropout = 0.0f, int64_t num_layers = 1, float resnet_eps = 1e-6f, int64_t resnet_groups = 32,
                     bool resnet_pre_norm = true, float output_scale_factor = 1.0f, bool add_upsample = true,
                     std::optional<int64_t> temb_channels = std::nullopt) {
        (void)resolution_idx;
        for (int64_t i = 0; i < num_layers; ++i) {
            resnets_.emplace_back(new ResnetBlock2D<SiLU>(i == 0 ? in_channels : out_channels, out_channels,
                                                          std::nullopt, dropout, temb_channels, resnet_groups,
                                                          std::nullopt, resnet_pre_norm, resnet_eps, false, 3,
                                                          output_scale_factor));
            register_module("resnets." + std::to_string(i), *resnets_.back());
        }
        if (add_upsample) {
            up_.reset(new Upsample2D(out_channels, true, out_channels));
            register_module("upsamplers.0", *up_);
        }
    }

    Tensor forward(Tensor hidden_states) const {
        for (const auto& r : resnets_) hidden_states = r->forward(hidden_states);
        return up_ ? up_->forward(hidden_states) : hidden_states;
    }

private:
    std::vector<std::unique_ptr<ResnetBlock2D<SiLU>>> resnets_;
    std::unique_ptr<Upsample2D> up_;
};

}  // namespace host
}  // namespace dit
