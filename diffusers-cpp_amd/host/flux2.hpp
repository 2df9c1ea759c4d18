// flux2.hpp -- the Flux2 transformer modules restated on the host Tensor
// layer, so that a full denoising step records the same node graph the
// reference records through its Runtime (Linear -> mul_mat, attention ->
// flash_attn_ext, the elementwise chain -> the fused kernels):
//   Linear                         src/nn/Linear.cpp:8-36
//   Timesteps                      src/diffusers/models/embeddings/Timesteps.cpp:6-45
//   TimestepEmbedding              src/diffusers/models/embeddings/TimestepEmbedding.inl:6-44
//   Flux2TimestepGuidanceEmbeddings  .../transformers/flux2/Flux2TimestepGuidanceEmbeddings.hpp:8-43
//   Flux2Modulation::forward       .../flux2/Flux2Modulation.hpp:10-22
//   ScaledDotProductAttention<FlashAttentionOp>
//                                  src/nn/attention/ScaledDotProductAttention.hpp:6-38,
//                                  src/nn/attention/FlashAttentionOp.cpp:6-105
//   Flux2Attention                 .../flux2/Flux2Attention.hpp:12-173
//   Flux2FeedForward               .../flux2/Flux2FeedForward.hpp:8-82
//   Flux2TransformerBlock          .../flux2/Flux2TransformerBlock.hpp:9-118
//   Flux2FusedQKVProjection        .../flux2/Flux2FusedQKVProjection.hpp:6-93
//   Flux2FusedAttentionOutput      .../flux2/Flux2FusedAttentionOutput.hpp:6-62
//   Flux2ParallelSelfAttention     .../flux2/Flux2ParallelSelfAttention.hpp:11-116
//   Flux2SingleTransformerBlock    .../flux2/Flux2SingleTransformerBlock.hpp:9-73
//   AdaLayerNormContinuous         src/diffusers/models/normalization/AdaLayerNormContinuous.inl:8-40
//   Flux2Transformer2DModel        .../flux2/Flux2Transformer2DModel.cpp:35-232
// Parameter names follow the reference's module tree.  Linear weights are
// created with the type set by LinearWeightType (F32 by default, as the
// reference's parameters; BF16 for the bf16 step).
#pragma once

#include <cmath>
#include <memory>
#include <optional>
#include <string>
#include <utility>
#include <vector>

#include "modules.hpp"

namespace dit {
namespace host {

inline int32_t& linear_weight_type_slot() {
    thread_local int32_t t = DT_TYPE_F32;
    return t;
}

// Scoped choice of the type new Linear weights are created with.
class LinearWeightType {
public:
    explicit LinearWeightType(int32_t type) : prev_(linear_weight_type_slot()) { linear_weight_type_slot() = type; }
    ~LinearWeightType() { linear_weight_type_slot() = prev_; }

private:
    int32_t prev_;
};

inline Tensor t_exp(const Tensor& t) { return Tensor(current_runtime().exp(*t), t.shape()); }
inline Tensor t_sin(const Tensor& t) { return Tensor(current_runtime().sin(*t), t.shape()); }
inline Tensor t_cos(const Tensor& t) { return Tensor(current_runtime().cos(*t), t.shape()); }

// Tensor::arange: an F32 leaf holding start, start + 1, ... (< end).
inline Tensor arange(float start, float end) {
    auto* hip = dynamic_cast<HipRuntime*>(&current_runtime());
    if (!hip) throw Unsupported("arange: needs a HipRuntime in scope");
    std::vector<float> v;
    for (float x = start; x < end; x += 1.0f) v.push_back(x);
    Tensor t = Tensor::empty({(int64_t)v.size()}, DT_TYPE_F32);
    hip->set_input(*t);
    hip->bind(*t, v.data(), v.size() * sizeof(float));
    return t;
}

class Linear : public Module {
public:
    Linear(int64_t in_features, int64_t out_features, bool bias = true) : out_(out_features), has_bias_(bias) {
        weight = parameter({out_features, in_features}, linear_weight_type_slot());
        register_parameter("weight", weight);
        if (bias) {
            this->bias = parameter({out_features});
            register_parameter("bias", this->bias);
        }
    }
    Tensor forward(const Tensor& x) const {
        Node* y = current_runtime().mul_mat(*weight, *x);
        if (has_bias_) y = current_runtime().add(y, *bias);
        Tensor::Shape shape = x.shape();
        shape.back() = out_;
        return Tensor(y, shape);
    }
    Tensor weight, bias;

private:
    int64_t out_;
    bool has_bias_;
};

class Timesteps : public Module {
public:
    Timesteps(int64_t num_channels, bool flip_sin_to_cos, float downscale_freq_shift = 1.0f, float scale = 1.0f)
        : channels_(num_channels), flip_(flip_sin_to_cos), shift_(downscale_freq_shift), scale_(scale) {}
    Tensor forward(const Tensor& timesteps) const {
        const int64_t half = channels_ / 2;
        Tensor exponent = arange(0.0f, (float)half);
        exponent = exponent * (-std::log(10000.0f) / ((float)half - shift_));
        Tensor emb = t_exp(exponent);
        emb = timesteps.unsqueeze(-1) * emb.unsqueeze(0);
        emb = emb * scale_;
        Tensor s = t_sin(emb), c = t_cos(emb);
        Tensor out = flip_ ? Tensor::cat({c, s}, -1) : Tensor::cat({s, c}, -1);
        if (channels_ % 2 == 1) throw Unsupported("Timesteps: odd channel counts are not supported");
        return out;
    }

private:
    int64_t channels_;
    bool flip_;
    float shift_, scale_;
};

class TimestepEmbedding : public Module {
public:
    TimestepEmbedding(int64_t in_channels, int64_t time_embed_dim, bool sample_proj_bias = true)
        : linear_1(in_channels, time_embed_dim, sample_proj_bias),
          linear_2(time_embed_dim, time_embed_dim, sample_proj_bias) {
        register_module("linear_1", linear_1);
        register_module("linear_2", linear_2);
    }
    Tensor forward(const Tensor& sample) const {
        return linear_2.forward(SiLU().forward(linear_1.forward(sample)));
    }
    Linear linear_1, linear_2;
};

class Flux2TimestepGuidanceEmbeddings : public Module {
public:
    Flux2TimestepGuidanceEmbeddings(int64_t in_channels, int64_t embedding_dim, bool bias, bool guidance_embeds)
        : time_proj(in_channels, true, 0.0f), timestep_embedder(in_channels, embedding_dim, bias) {
        register_module("timestep_embedder", timestep_embedder);
        if (guidance_embeds) {
            guidance_embedder = std::make_unique<TimestepEmbedding>(in_channels, embedding_dim, bias);
            register_module("guidance_embedder", *guidance_embedder);
        }
    }
    Tensor forward(const Tensor& timestep, const std::optional<Tensor>& guidance) const {
        Tensor emb = timestep_embedder.forward(time_proj.forward(timestep));
        if (guidance_embedder) {
            if (!guidance) throw std::invalid_argument("Flux2TimestepGuidanceEmbeddings: guidance required");
            emb = emb + guidance_embedder->forward(time_proj.forward(*guidance));
        }
        return emb;
    }
    Timesteps time_proj;
    TimestepEmbedding timestep_embedder;
    std::unique_ptr<TimestepEmbedding> guidance_embedder;
};

class Flux2ModulationLayer : public Module {
public:
    Flux2ModulationLayer(int64_t dim, int64_t mod_param_sets, bool bias = false)
        : linear(dim, dim * 3 * mod_param_sets, bias) {
        register_module("linear", linear);
    }
    Tensor forward(const Tensor& temb) const { return linear.forward(SiLU().forward(temb)); }
    Linear linear;
};

// ScaledDotProductAttention<FlashAttentionOp>: [B, S, H, D] in and out.
inline Tensor scaled_dot_product_attention(const Tensor& query, const Tensor& key, const Tensor& value) {
    Tensor q = query.transpose(1, 2), k = key.transpose(1, 2), v = value.transpose(1, 2);
    const float scale = 1.0f / std::sqrt((float)q.shape().back());
    Tensor::Shape shape = q.shape();  // (B, H, S, D) -> ggml output (B, S, H, D)
    std::swap(shape[1], shape[2]);
    Tensor attn(current_runtime().flash_attn_ext(*q, *k, *v, nullptr, scale, 0.0f, 0.0f), shape);
    attn = attn.permute({0, 2, 1, 3});
    return attn.transpose(1, 2);
}

using RotaryEmb = std::pair<const Flux2PosEmbed*, Tensor>;

class Flux2Attention : public Module {
public:
    Flux2Attention(int64_t query_dim, int64_t heads, int64_t dim_head, bool bias, int64_t added_kv_proj_dim,
                   bool added_proj_bias, bool out_bias, float eps, int64_t out_dim)
        : heads_(out_dim / dim_head),
          to_q(query_dim, out_dim, bias), to_k(query_dim, out_dim, bias), to_v(query_dim, out_dim, bias),
          norm_q(dim_head, eps, true), norm_k(dim_head, eps, true), to_out_0(out_dim, out_dim, out_bias),
          norm_added_q(dim_head, eps), norm_added_k(dim_head, eps),
          add_q_proj(added_kv_proj_dim, out_dim, added_proj_bias),
          add_k_proj(added_kv_proj_dim, out_dim, added_proj_bias),
          add_v_proj(added_kv_proj_dim, out_dim, added_proj_bias), to_add_out(out_dim, query_dim, out_bias) {
        (void)heads;
        register_module("to_q", to_q);
        register_module("to_k", to_k);
        register_module("to_v", to_v);
        register_module("norm_q", norm_q);
        register_module("norm_k", norm_k);
        register_module("to_out.0", to_out_0);
        register_module("norm_added_q", norm_added_q);
        register_module("norm_added_k", norm_added_k);
        register_module("add_q_proj", add_q_proj);
        register_module("add_k_proj", add_k_proj);
        register_module("add_v_proj", add_v_proj);
        register_module("to_add_out", to_add_out);
    }
    // -> {hidden_states, encoder_hidden_states}
    std::pair<Tensor, Tensor> forward(const Tensor& hidden_states, const Tensor& encoder_hidden_states,
                                      const RotaryEmb& rotary) const {
        Tensor query = to_q.forward(hidden_states);
        Tensor key = to_k.forward(hidden_states);
        Tensor value = to_v.forward(hidden_states);
        Tensor eq = add_q_proj.forward(encoder_hidden_states);
        Tensor ek = add_k_proj.forward(encoder_hidden_states);
        Tensor ev = add_v_proj.forward(encoder_hidden_states);
        query = norm_q.forward(query.unflatten(-1, {heads_, -1}));
        key = norm_k.forward(key.unflatten(-1, {heads_, -1}));
        value = value.unflatten(-1, {heads_, -1});
        eq = norm_added_q.forward(eq.unflatten(-1, {heads_, -1}));
        ek = norm_added_k.forward(ek.unflatten(-1, {heads_, -1}));
        ev = ev.unflatten(-1, {heads_, -1});
        query = Tensor::cat({eq, query}, 1);
        key = Tensor::cat({ek, key}, 1);
        value = Tensor::cat({ev, value}, 1);
        query = rotary.first->forward(query, rotary.second);
        key = rotary.first->forward(key, rotary.second);
        Tensor h = scaled_dot_product_attention(query, key, value).flatten(2, 3);
        const int64_t n_txt = encoder_hidden_states.shape()[1];
        Tensor enc = h.narrow(1, 0, n_txt);
        h = h.narrow(1, n_txt, h.shape()[1] - n_txt);
        return {to_out_0.forward(h), to_add_out.forward(enc)};
    }

    int64_t heads_;
    Linear to_q, to_k, to_v;
    RMSNorm norm_q, norm_k;
    Linear to_out_0;
    RMSNorm norm_added_q, norm_added_k;
    Linear add_q_proj, add_k_proj, add_v_proj, to_add_out;
};

class Flux2FeedForward : public Module {
public:
    Flux2FeedForward(int64_t dim, int64_t dim_out, float mult, bool bias)
        : linear_in_gate(dim, (int64_t)(dim * mult), bias), linear_in_up(dim, (int64_t)(dim * mult), bias),
          linear_out((int64_t)(dim * mult), dim_out, bias) {
        register_module("linear_in_gate", linear_in_gate);
        register_module("linear_in_up", linear_in_up);
        register_module("linear_out", linear_out);
    }
    Tensor forward(const Tensor& x) const {
        Tensor gate = linear_in_gate.forward(x);
        Tensor up = linear_in_up.forward(x);
        return linear_out.forward(Flux2SwiGLU().forward(gate, up));
    }
    Linear linear_in_gate, linear_in_up, linear_out;
};

class Flux2TransformerBlock : public Module {
public:
    Flux2TransformerBlock(int64_t dim, int64_t heads, int64_t head_dim, float mlp_ratio, float eps, bool bias)
        : norm1(dim, eps, false), norm1_context(dim, eps, false),
          attn(dim, heads, head_dim, bias, dim, bias, bias, eps, dim), norm2(dim, eps, false),
          ff(dim, dim, mlp_ratio, bias), norm2_context(dim, eps, false), ff_context(dim, dim, mlp_ratio, bias) {
        register_module("attn", attn);
        register_module("ff", ff);
        register_module("ff_context", ff_context);
    }
    // -> {encoder_hidden_states, hidden_states}
    std::pair<Tensor, Tensor> forward(Tensor hidden_states, Tensor encoder_hidden_states, const Tensor& temb_mod_img,
                                      const Tensor& temb_mod_txt, const RotaryEmb& rotary) const {
        auto img = Flux2Modulation::split(temb_mod_img, 2);
        auto txt = Flux2Modulation::split(temb_mod_txt, 2);
        const Tensor &shift_msa = img[0][0], &scale_msa = img[0][1], &gate_msa = img[0][2];
        const Tensor &shift_mlp = img[1][0], &scale_mlp = img[1][1], &gate_mlp = img[1][2];
        const Tensor &c_shift_msa = txt[0][0], &c_scale_msa = txt[0][1], &c_gate_msa = txt[0][2];
        const Tensor &c_shift_mlp = txt[1][0], &c_scale_mlp = txt[1][1], &c_gate_mlp = txt[1][2];

        Tensor norm_h = (1.0f + scale_msa) * norm1.forward(hidden_states) + shift_msa;
        Tensor norm_e = (1.0f + c_scale_msa) * norm1_context.forward(encoder_hidden_states) + c_shift_msa;
        auto [attn_output, context_attn_output] = attn.forward(norm_h, norm_e, rotary);

        hidden_states = hidden_states + gate_msa * attn_output;
        norm_h = norm2.forward(hidden_states) * (1.0f + scale_mlp) + shift_mlp;
        hidden_states = hidden_states + gate_mlp * ff.forward(norm_h);

        encoder_hidden_states = encoder_hidden_states + c_gate_msa * context_attn_output;
        norm_e = norm2_context.forward(encoder_hidden_states) * (1.0f + c_scale_mlp) + c_shift_mlp;
        encoder_hidden_states = encoder_hidden_states + c_gate_mlp * ff_context.forward(norm_e);
        return {encoder_hidden_states, hidden_states};
    }

    LayerNorm norm1, norm1_context;
    Flux2Attention attn;
    LayerNorm norm2;
    Flux2FeedForward ff;
    LayerNorm norm2_context;
    Flux2FeedForward ff_context;
};

class Flux2ParallelSelfAttention : public Module {
public:
    Flux2ParallelSelfAttention(int64_t query_dim, int64_t heads, int64_t dim_head, bool bias, bool out_bias,
                               float eps, int64_t out_dim, float mlp_ratio)
        : heads_(out_dim / dim_head), mlp_hidden_(int64_t(query_dim * mlp_ratio)),
          q(query_dim, out_dim, bias), k(query_dim, out_dim, bias), v(query_dim, out_dim, bias),
          mlp_in_gate(query_dim, mlp_hidden_, bias), mlp_in_up(query_dim, mlp_hidden_, bias),
          norm_q(dim_head, eps, true), norm_k(dim_head, eps, true),
          out_attn(out_dim, out_dim, out_bias), out_mlp(mlp_hidden_, out_dim, false) {
        (void)heads;
        register_module("to_qkv_mlp_proj.q", q);
        register_module("to_qkv_mlp_proj.k", k);
        register_module("to_qkv_mlp_proj.v", v);
        register_module("to_qkv_mlp_proj.mlp_in_gate", mlp_in_gate);
        register_module("to_qkv_mlp_proj.mlp_in_up", mlp_in_up);
        register_module("norm_q", norm_q);
        register_module("norm_k", norm_k);
        register_module("to_out.attn", out_attn);
        register_module("to_out.mlp", out_mlp);
    }
    Tensor forward(const Tensor& hidden_states, const RotaryEmb& rotary) const {
        Tensor query = q.forward(hidden_states);
        Tensor key = k.forward(hidden_states);
        Tensor value = v.forward(hidden_states);
        Tensor gate = mlp_in_gate.forward(hidden_states);
        Tensor up = mlp_in_up.forward(hidden_states);
        query = norm_q.forward(query.unflatten(-1, {heads_, -1}));
        key = norm_k.forward(key.unflatten(-1, {heads_, -1}));
        value = value.unflatten(-1, {heads_, -1});
        query = rotary.first->forward(query, rotary.second);
        key = rotary.first->forward(key, rotary.second);
        Tensor h = scaled_dot_product_attention(query, key, value).flatten(2, 3);
        Tensor mlp = Flux2SwiGLU().forward(gate, up);
        // Flux2FusedAttentionOutput::forward: attn(h) + mlp(m)
        return out_attn.forward(h) + out_mlp.forward(mlp);
    }

    int64_t heads_, mlp_hidden_;
    Linear q, k, v, mlp_in_gate, mlp_in_up;
    RMSNorm norm_q, norm_k;
    Linear out_attn, out_mlp;
};

class Flux2SingleTransformerBlock : public Module {
public:
    Flux2SingleTransformerBlock(int64_t dim, int64_t heads, int64_t head_dim, float mlp_ratio, float eps, bool bias)
        : norm(dim, eps, false), attn(dim, heads, head_dim, bias, bias, eps, dim, mlp_ratio) {
        register_module("attn", attn);
    }
    Tensor forward(Tensor hidden_states, const Tensor& temb_mod, const RotaryEmb& rotary) const {
        auto m = Flux2Modulation::split(temb_mod, 1)[0];
        Tensor norm_h = (1.0f + m[1]) * norm.forward(hidden_states) + m[0];
        Tensor attn_output = attn.forward(norm_h, rotary);
        return hidden_states + m[2] * attn_output;
    }

    LayerNorm norm;
    Flux2ParallelSelfAttention attn;
};

class AdaLayerNormContinuous : public Module {
public:
    AdaLayerNormContinuous(int64_t embedding_dim, int64_t conditioning_embedding_dim, float eps)
        : linear(conditioning_embedding_dim, embedding_dim * 2, false), norm(embedding_dim, eps, false, false) {
        register_module("linear", linear);
    }
    Tensor forward(const Tensor& hidden_states, const Tensor& conditioning_embedding) const {
        Tensor emb = linear.forward(SiLU().forward(conditioning_embedding));
        auto parts = emb.chunk(2, 1);
        const Tensor& scale = parts.at(0);
        const Tensor& shift = parts.at(1);
        return norm.forward(hidden_states) * (1.0f + scale).unsqueeze(1) + shift.unsqueeze(1);
    }
    Linear linear;
    LayerNorm norm;
};

// Flux2Transformer2DModel::Config (Flux2Transformer2DModel.hpp:12-31).
struct Flux2Config {
    int64_t patch_size = 1;
    int64_t in_channels = 128;
    int64_t out_channels = 128;
    int64_t num_layers = 8;
    int64_t num_single_layers = 48;
    int64_t attention_head_dim = 128;
    int64_t num_attention_heads = 48;
    int64_t joint_attention_dim = 15360;
    int64_t timestep_guidance_channels = 256;
    float mlp_ratio = 3.0f;
    std::vector<int64_t> axes_dims_rope = {32, 32, 32, 32};
    int64_t rope_theta = 2000;
    float eps = 1e-6f;
    bool guidance_embeds = true;
};

class Flux2Transformer2DModel : public Module {
public:
    explicit Flux2Transformer2DModel(const Flux2Config& c)
        : inner_(c.num_attention_heads * c.attention_head_dim),
          pos_embed(c.rope_theta, c.axes_dims_rope),
          time_guidance_embed(c.timestep_guidance_channels, inner_, false, c.guidance_embeds),
          double_stream_modulation_img(inner_, 2), double_stream_modulation_txt(inner_, 2),
          single_stream_modulation(inner_, 1), x_embedder(c.in_channels, inner_, false),
          context_embedder(c.joint_attention_dim, inner_, false), norm_out(inner_, inner_, c.eps),
          proj_out(inner_, c.patch_size * c.patch_size * c.out_channels, false) {
        register_module("time_guidance_embed", time_guidance_embed);
        register_module("double_stream_modulation_img", double_stream_modulation_img);
        register_module("double_stream_modulation_txt", double_stream_modulation_txt);
        register_module("single_stream_modulation", single_stream_modulation);
        register_module("x_embedder", x_embedder);
        register_module("context_embedder", context_embedder);
        for (int64_t i = 0; i < c.num_layers; ++i) {
            transformer_blocks.push_back(std::make_unique<Flux2TransformerBlock>(
                inner_, c.num_attention_heads, c.attention_head_dim, c.mlp_ratio, c.eps, false));
            register_module("transformer_blocks." + std::to_string(i), *transformer_blocks.back());
        }
        for (int64_t i = 0; i < c.num_single_layers; ++i) {
            single_transformer_blocks.push_back(std::make_unique<Flux2SingleTransformerBlock>(
                inner_, c.num_attention_heads, c.attention_head_dim, c.mlp_ratio, c.eps, false));
            register_module("single_transformer_blocks." + std::to_string(i), *single_transformer_blocks.back());
        }
        register_module("norm_out", norm_out);
        register_module("proj_out", proj_out);
    }

    // hidden_states [1, N_img, in_channels], encoder_hidden_states [1, N_txt,
    // joint_attention_dim], timestep [1] (F32), img_ids [N_img, 4] and
    // txt_ids [N_txt, 4] (I32) -> [1, N_img, out_channels].
    Tensor forward(Tensor hidden_states, Tensor encoder_hidden_states, Tensor timestep, const Tensor& img_ids,
                   const Tensor& txt_ids, std::optional<Tensor> guidance = std::nullopt) const {
        const int64_t num_txt = encoder_hidden_states.shape()[1];
        timestep = timestep * 1000.0f;
        if (guidance) guidance = *guidance * 1000.0f;
        Tensor temb = time_guidance_embed.forward(timestep, guidance);
        Tensor mod_img = double_stream_modulation_img.forward(temb);
        Tensor mod_txt = double_stream_modulation_txt.forward(temb);
        Tensor mod_single = single_stream_modulation.forward(temb);

        hidden_states = x_embedder.forward(hidden_states);
        encoder_hidden_states = context_embedder.forward(encoder_hidden_states);
        const RotaryEmb rotary{&pos_embed, Tensor::cat({txt_ids, img_ids}, 0)};

        for (const auto& block : transformer_blocks) {
            auto [enc, hid] = block->forward(hidden_states, encoder_hidden_states, mod_img, mod_txt, rotary);
            encoder_hidden_states = enc;
            hidden_states = hid;
        }
        hidden_states = Tensor::cat({encoder_hidden_states, hidden_states}, 1);
        for (const auto& block : single_transformer_blocks)
            hidden_states = block->forward(hidden_states, mod_single, rotary);
        hidden_states = hidden_states.narrow(1, num_txt, hidden_states.shape()[1] - num_txt);
        hidden_states = norm_out.forward(hidden_states, temb);
        return proj_out.forward(hidden_states);
    }

    int64_t inner_;
    Flux2PosEmbed pos_embed;
    Flux2TimestepGuidanceEmbeddings time_guidance_embed;
    Flux2ModulationLayer double_stream_modulation_img, double_stream_modulation_txt, single_stream_modulation;
    Linear x_embedder, context_embedder;
    std::vector<std::unique_ptr<Flux2TransformerBlock>> transformer_blocks;
    std::vector<std::unique_ptr<Flux2SingleTransformerBlock>> single_transformer_blocks;
    AdaLayerNormContinuous norm_out;
    Linear proj_out;
};

}  // namespace host
}  // namespace dit
