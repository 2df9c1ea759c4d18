"""VAE decoder blocks composed from the oracle's fp32 ops.

Test infrastructure only (the tests use it as the checker); the product
never imports it.  Each function follows the reference module it names, op
for op, in fp32 with NCHW tensors:

  resnet_block2d      ResnetBlock2D::forward
                      (src/diffusers/models/resnet/ResnetBlock2D.inl:7-195)
  up_decoder_block2d  UpDecoderBlock2D::forward
                      (src/diffusers/models/unets/unet2d/UpDecoderBlock2D.cpp:6-74)

Parameters are a dict keyed by the reference's dotted parameter paths
(norm1.weight, conv1.bias, ...); resnet_block2d_param_shapes lists them.
"""
from __future__ import annotations

import numpy as np

from . import conv2d, groupnorm_silu, linear, round_bf16, sigmoid


def resnet_block2d_param_shapes(in_channels: int, out_channels: int | None = None,
                                temb_channels: int | None = None, kernel_size: int = 3,
                                use_in_shortcut: bool | None = None, conv_shortcut_bias: bool = True,
                                conv_2d_out_channels: int | None = None, prefix: str = ""):
    """The block's parameters as the constructor creates them
    (ResnetBlock2D.inl:27-100): norm1 over in_channels, conv1 in -> out,
    time_emb_proj only with temb_channels, norm2 and conv2 out -> conv2d_out,
    and a 1x1 conv_shortcut when in_channels differs from conv2d_out (or
    use_in_shortcut says so)."""
    out = out_channels if out_channels is not None else in_channels
    c2 = conv_2d_out_channels if conv_2d_out_channels is not None else out
    k = kernel_size
    s = {
        "norm1.weight": (in_channels,), "norm1.bias": (in_channels,),
        "conv1.weight": (out, in_channels, k, k), "conv1.bias": (out,),
        "norm2.weight": (out,), "norm2.bias": (out,),
        "conv2.weight": (c2, out, k, k), "conv2.bias": (c2,),
    }
    if temb_channels is not None:
        s["time_emb_proj.weight"] = (out, temb_channels)
        s["time_emb_proj.bias"] = (out,)
    if (use_in_shortcut if use_in_shortcut is not None else in_channels != c2):
        s["conv_shortcut.weight"] = (c2, in_channels, 1, 1)
        if conv_shortcut_bias:
            s["conv_shortcut.bias"] = (c2,)
    return {prefix + n: v for n, v in s.items()}


def _silu(x):
    """SiLU module: x * sigmoid(x) (src/nn/SiLU.hpp:9-13), two fp32 roundings."""
    x = np.asarray(x, np.float32)
    return (x * sigmoid(x)).astype(np.float32)


def resnet_block2d(x, P, groups=32, groups_out=None, eps=1e-6, output_scale_factor=1.0, temb=None,
                   prefix="", threads=0, conv_bf16=False):
    """ResnetBlock2D::forward (ResnetBlock2D.inl:110-195), pre_norm, no
    up/down sampling.  x: [N, Cin, H, W]; temb: [N, temb_channels] or None.

    norm1 -> SiLU -> conv1, then (with time_emb_proj and temb) + the
    projected SiLU(temb) broadcast over H and W (inl:129-161), norm2 ->
    SiLU -> conv2; the shortcut is conv_shortcut(x) when the block has one
    (inl:188-192); the result is (x + h) scaled by 1 / output_scale_factor,
    a ggml_scale of the fp32 reciprocal as Tensor / float records it
    (src/ggml/Tensor.hpp:366-369).

    conv_bf16 rounds each convolution's input and weight to bf16 first, the
    operand precision of an MFMA convolution with fp32 accumulation."""
    g = lambda n: P[prefix + n]
    conv = conv2d
    if conv_bf16:
        conv = lambda a, w, b, padding, threads: conv2d(round_bf16(a), round_bf16(w), b, padding=padding,
                                                        threads=threads)
    has = lambda n: (prefix + n) in P
    x = np.asarray(x, np.float32)
    k1 = g("conv1.weight").shape[-1]
    h = groupnorm_silu(x, groups, g("norm1.weight"), g("norm1.bias"), eps, threads=threads)
    h = conv(h, g("conv1.weight"), g("conv1.bias"), padding=k1 // 2, threads=threads)
    if has("time_emb_proj.weight") and temb is not None:
        t = linear(_silu(temb), g("time_emb_proj.weight"), g("time_emb_proj.bias"), threads=threads)
        h = (h + t[:, :, None, None]).astype(np.float32)
    k2 = g("conv2.weight").shape[-1]
    h = groupnorm_silu(h, groups_out if groups_out is not None else groups, g("norm2.weight"), g("norm2.bias"),
                       eps, threads=threads)
    h = conv(h, g("conv2.weight"), g("conv2.bias"), padding=k2 // 2, threads=threads)
    if has("conv_shortcut.weight"):
        x = conv(x, g("conv_shortcut.weight"), P.get(prefix + "conv_shortcut.bias"), padding=0, threads=threads)
    s = (x + h).astype(np.float32)
    return (s * (np.float32(1.0) / np.float32(output_scale_factor))).astype(np.float32)


def up_decoder_block2d_param_shapes(in_channels: int, out_channels: int, num_layers: int = 1,
                                    add_upsample: bool = True, temb_channels: int | None = None,
                                    prefix: str = ""):
    """UpDecoderBlock2D's parameters (UpDecoderBlock2D.cpp:20-57): resnets.<i>.*
    (the first in -> out, the rest out -> out) and upsamplers.0.conv.*."""
    s = {}
    for i in range(num_layers):
        s.update(resnet_block2d_param_shapes(in_channels if i == 0 else out_channels, out_channels, temb_channels,
                                             prefix=f"{prefix}resnets.{i}."))
    if add_upsample:
        s[f"{prefix}upsamplers.0.conv.weight"] = (out_channels, out_channels, 3, 3)
        s[f"{prefix}upsamplers.0.conv.bias"] = (out_channels,)
    return s


def up_decoder_block2d(x, P, num_layers=1, resnet_groups=32, eps=1e-6, output_scale_factor=1.0,
                       add_upsample=True, prefix="", threads=0, conv_bf16=False):
    """UpDecoderBlock2D::forward (UpDecoderBlock2D.cpp:60-74): the resnets in
    order (temb is not passed to them), then with add_upsample the
    Upsample2D: nearest 2x and its 3x3 conv + bias (Upsample2D.cpp:36-63)."""
    h = np.asarray(x, np.float32)
    for i in range(num_layers):
        h = resnet_block2d(h, P, resnet_groups, None, eps, output_scale_factor, None, prefix=f"{prefix}resnets.{i}.",
                           threads=threads, conv_bf16=conv_bf16)
    if add_upsample:
        w = P[prefix + "upsamplers.0.conv.weight"]
        b = P[prefix + "upsamplers.0.conv.bias"]
        if conv_bf16:
            h, w = round_bf16(h), round_bf16(w)
        h = conv2d(h, w, b, up2=True, threads=threads)
    return h
