"""Flux2 transformer forward passes composed from the oracle's fp32 ops.

Test infrastructure only (the tests, the smoke check and the benchmark's CPU
baseline use it, as the checker or as the timed CPU path); the product never
imports it.  Each function follows the reference module it names, op for op,
in fp32 with batch 1 (tokens are rows):

  single_block   Flux2SingleTransformerBlock::forward
                 (src/diffusers/models/transformers/flux2/Flux2SingleTransformerBlock.hpp:36-72,
                 Flux2ParallelSelfAttention.hpp:55-101, Flux2FusedAttentionOutput.hpp:31-36)
  double_block   Flux2TransformerBlock::forward (Flux2TransformerBlock.hpp:47-116,
                 Flux2Attention.hpp:57-160, Flux2FeedForward.hpp:62-72)
  model          Flux2Transformer2DModel::forward (Flux2Transformer2DModel.cpp:109-232)

Parameters are a dict keyed by the reference's dotted parameter paths; the
*_param_shapes functions list them.  Linear weights are [out, in].
"""
from __future__ import annotations

import numpy as np

from . import (adaln, attention, concat, gated_residual, linear, norm, qk_rmsnorm_rope, sigmoid,
               swiglu)


# ---- parameter inventories ----------------------------------------------------

def single_block_param_shapes(dim: int, heads: int, mlp_ratio: float = 3.0, prefix: str = ""):
    hd, mlp = dim // heads, int(dim * mlp_ratio)
    p = prefix + "attn."
    return {
        p + "to_qkv_mlp_proj.q.weight": (dim, dim),
        p + "to_qkv_mlp_proj.k.weight": (dim, dim),
        p + "to_qkv_mlp_proj.v.weight": (dim, dim),
        p + "to_qkv_mlp_proj.mlp_in_gate.weight": (mlp, dim),
        p + "to_qkv_mlp_proj.mlp_in_up.weight": (mlp, dim),
        p + "norm_q.weight": (hd,),
        p + "norm_k.weight": (hd,),
        p + "to_out.attn.weight": (dim, dim),
        p + "to_out.mlp.weight": (dim, mlp),
    }


def double_block_param_shapes(dim: int, heads: int, mlp_ratio: float = 3.0, prefix: str = ""):
    hd, mlp = dim // heads, int(dim * mlp_ratio)
    a = prefix + "attn."
    s = {}
    for n in ("to_q", "to_k", "to_v", "to_out.0", "add_q_proj", "add_k_proj", "add_v_proj", "to_add_out"):
        s[a + n + ".weight"] = (dim, dim)
    for n in ("norm_q", "norm_k", "norm_added_q", "norm_added_k"):
        s[a + n + ".weight"] = (hd,)
    for ff in ("ff", "ff_context"):
        s[prefix + ff + ".linear_in_gate.weight"] = (mlp, dim)
        s[prefix + ff + ".linear_in_up.weight"] = (mlp, dim)
        s[prefix + ff + ".linear_out.weight"] = (dim, mlp)
    return s


def model_param_shapes(cfg: dict):
    d = cfg["num_attention_heads"] * cfg["attention_head_dim"]
    heads, r = cfg["num_attention_heads"], cfg.get("mlp_ratio", 3.0)
    tc = cfg.get("timestep_guidance_channels", 256)
    s = {
        "time_guidance_embed.timestep_embedder.linear_1.weight": (d, tc),
        "time_guidance_embed.timestep_embedder.linear_2.weight": (d, d),
        "double_stream_modulation_img.linear.weight": (6 * d, d),
        "double_stream_modulation_txt.linear.weight": (6 * d, d),
        "single_stream_modulation.linear.weight": (3 * d, d),
        "x_embedder.weight": (d, cfg["in_channels"]),
        "context_embedder.weight": (d, cfg["joint_attention_dim"]),
    }
    for i in range(cfg["num_layers"]):
        s.update(double_block_param_shapes(d, heads, r, f"transformer_blocks.{i}."))
    for i in range(cfg["num_single_layers"]):
        s.update(single_block_param_shapes(d, heads, r, f"single_transformer_blocks.{i}."))
    s["norm_out.linear.weight"] = (2 * d, d)
    s["proj_out.weight"] = (cfg["in_channels"], d)
    return s


# ---- pieces ---------------------------------------------------------------------

def silu(x):
    """SiLU module: x * sigmoid(x) (src/nn/SiLU.hpp:9-13), two fp32 roundings."""
    x = np.asarray(x, np.float32)
    return (x * sigmoid(x)).astype(np.float32)


def _split_mod(mod, sets):
    """Flux2Modulation::split (Flux2Modulation.hpp:24-41): 3*sets chunks of the last dim."""
    m = np.asarray(mod, np.float32).reshape(-1)
    d = m.size // (3 * sets)
    return [[m[(3 * i + j) * d:(3 * i + j + 1) * d] for j in range(3)] for i in range(sets)]


def _adaln_mul_first(x, shift, scale, eps):
    """`norm(x) * (1 + scale) + shift` (Flux2TransformerBlock.hpp:91-92): the
    same two roundings as adaln's `(1 + scale) * norm(x) + shift`."""
    return adaln(x, shift, scale, eps)


def _qk(x, w, pos, heads, axes_dim, theta, eps, threads=0):
    S = x.shape[0]
    return qk_rmsnorm_rope(x.reshape(S, heads, -1), w, pos, axes_dim, theta, eps, threads)


def timestep_proj(t, channels=256, flip_sin_to_cos=True, shift=0.0):
    """Timesteps::forward (src/diffusers/models/embeddings/Timesteps.cpp:17-45) in fp32."""
    half = channels // 2
    exponent = (np.arange(half, dtype=np.float32) * np.float32(-np.log(10000.0) / (half - shift))).astype(np.float32)
    emb = np.exp(exponent).astype(np.float32)
    emb = (np.float32(t) * emb).astype(np.float32)[None, :]
    s, c = np.sin(emb).astype(np.float32), np.cos(emb).astype(np.float32)
    return np.concatenate([c, s] if flip_sin_to_cos else [s, c], axis=-1)


# ---- blocks ---------------------------------------------------------------------

def single_block(x, temb_mod, pos, P, heads, theta, axes_dim=32, eps=1e-6, prefix="", threads=0):
    """x [S, D], temb_mod [3D], pos int32 [S, 4] -> [S, D] (threads: OpenMP
    threads of every op, 0 = all)."""
    x = np.asarray(x, np.float32)
    S, D = x.shape
    a = prefix + "attn."
    t = threads
    shift, scale, gate = _split_mod(temb_mod, 1)[0]
    n = adaln(x, shift, scale, eps, t)
    q = linear(n, P[a + "to_qkv_mlp_proj.q.weight"], threads=t)
    k = linear(n, P[a + "to_qkv_mlp_proj.k.weight"], threads=t)
    v = linear(n, P[a + "to_qkv_mlp_proj.v.weight"], threads=t)
    g = linear(n, P[a + "to_qkv_mlp_proj.mlp_in_gate.weight"], threads=t)
    u = linear(n, P[a + "to_qkv_mlp_proj.mlp_in_up.weight"], threads=t)
    q = _qk(q, P[a + "norm_q.weight"], pos, heads, axes_dim, theta, eps, t)
    k = _qk(k, P[a + "norm_k.weight"], pos, heads, axes_dim, theta, eps, t)
    o = attention(q, k, v.reshape(S, heads, -1), threads=t).reshape(S, D)
    m = swiglu(g, u, t)
    y = (linear(o, P[a + "to_out.attn.weight"], threads=t) +
         linear(m, P[a + "to_out.mlp.weight"], threads=t)).astype(np.float32)
    return gated_residual(x, y, gate, t)


def double_block(h, e, mod_img, mod_txt, pos, P, heads, theta, axes_dim=32, eps=1e-6, prefix=""):
    """h [S_img, D], e [S_txt, D]; pos int32 [S_txt + S_img, 4] (txt first) -> (e', h')."""
    h = np.asarray(h, np.float32)
    e = np.asarray(e, np.float32)
    n_txt, D = e.shape
    a = prefix + "attn."
    (sh, sc, gt), (sh2, sc2, gt2) = _split_mod(mod_img, 2)
    (csh, csc, cgt), (csh2, csc2, cgt2) = _split_mod(mod_txt, 2)
    nh = adaln(h, sh, sc, eps)
    ne = adaln(e, csh, csc, eps)
    q = linear(nh, P[a + "to_q.weight"])
    k = linear(nh, P[a + "to_k.weight"])
    v = linear(nh, P[a + "to_v.weight"])
    eq = linear(ne, P[a + "add_q_proj.weight"])
    ek = linear(ne, P[a + "add_k_proj.weight"])
    ev = linear(ne, P[a + "add_v_proj.weight"])
    # RMSNorm per stream, concatenated txt first, then RoPE over the joint sequence
    # (Flux2Attention.hpp:93-122): per-row ops, so normalising each stream with
    # its own weight and rotating by its own rows of `pos` is the same thing.
    qj = np.concatenate([_qk(eq, P[a + "norm_added_q.weight"], pos[:n_txt], heads, axes_dim, theta, eps),
                         _qk(q, P[a + "norm_q.weight"], pos[n_txt:], heads, axes_dim, theta, eps)])
    kj = np.concatenate([_qk(ek, P[a + "norm_added_k.weight"], pos[:n_txt], heads, axes_dim, theta, eps),
                         _qk(k, P[a + "norm_k.weight"], pos[n_txt:], heads, axes_dim, theta, eps)])
    vj = np.concatenate([ev, v]).reshape(qj.shape)
    o = attention(qj, kj, vj).reshape(-1, D)
    attn_out = linear(o[n_txt:], P[a + "to_out.0.weight"])
    ctx_out = linear(o[:n_txt], P[a + "to_add_out.weight"])

    h = gated_residual(h, attn_out, gt)
    nh = _adaln_mul_first(h, sh2, sc2, eps)
    ff = linear(swiglu(linear(nh, P[prefix + "ff.linear_in_gate.weight"]),
                       linear(nh, P[prefix + "ff.linear_in_up.weight"])), P[prefix + "ff.linear_out.weight"])
    h = gated_residual(h, ff, gt2)

    e = gated_residual(e, ctx_out, cgt)
    ne = _adaln_mul_first(e, csh2, csc2, eps)
    ffc = linear(swiglu(linear(ne, P[prefix + "ff_context.linear_in_gate.weight"]),
                        linear(ne, P[prefix + "ff_context.linear_in_up.weight"])),
                 P[prefix + "ff_context.linear_out.weight"])
    e = gated_residual(e, ffc, cgt2)
    return e, h


def model(hidden, text, timestep, img_ids, txt_ids, P, cfg):
    """hidden [N_img, in_channels], text [N_txt, joint_attention_dim] -> [N_img, in_channels]."""
    heads = cfg["num_attention_heads"]
    theta = float(cfg.get("rope_theta", 2000))
    axes = cfg.get("axes_dims_rope", [32, 32, 32, 32])
    assert len(set(axes)) == 1
    axis_dim = axes[0]
    eps = cfg.get("eps", 1e-6)
    t = np.float32(np.float32(timestep) * np.float32(1000.0))
    tp = timestep_proj(t, cfg.get("timestep_guidance_channels", 256))
    temb = linear(silu(linear(tp, P["time_guidance_embed.timestep_embedder.linear_1.weight"])),
                  P["time_guidance_embed.timestep_embedder.linear_2.weight"])
    st = silu(temb)
    mod_img = linear(st, P["double_stream_modulation_img.linear.weight"])
    mod_txt = linear(st, P["double_stream_modulation_txt.linear.weight"])
    mod_single = linear(st, P["single_stream_modulation.linear.weight"])
    h = linear(hidden, P["x_embedder.weight"])
    e = linear(text, P["context_embedder.weight"])
    pos = np.concatenate([txt_ids, img_ids]).astype(np.int32)
    for i in range(cfg["num_layers"]):
        e, h = double_block(h, e, mod_img, mod_txt, pos, P, heads, theta, axis_dim, eps,
                            f"transformer_blocks.{i}.")
    x = np.concatenate([e, h])
    for i in range(cfg["num_single_layers"]):
        x = single_block(x, mod_single, pos, P, heads, theta, axis_dim, eps, f"single_transformer_blocks.{i}.")
    x = x[e.shape[0]:]
    emb = linear(silu(temb), P["norm_out.linear.weight"]).reshape(-1)
    d = emb.size // 2
    x = adaln(x, emb[d:], emb[:d], eps)   # scale = first chunk, shift = second (AdaLayerNormContinuous.inl:30-38)
    return linear(x, P["proj_out.weight"])
