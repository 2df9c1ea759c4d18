"""Pins for the oracle's ResnetBlock2D composition (oracle/vae.py) on the CPU.

The block is checked against torch's own float64 group_norm / conv2d / linear
composed as the diffusers module the reference's test compares with
(test/src/diffusers/models/resnet/ResnetBlock2D.py: the default 8 -> 8 block,
the 8 -> 16 channel projection and the temb case, all groups 8 on a 2x2
input), and against closed forms a composition mistake would break: a zero
conv2 leaves exactly the (projected) shortcut times 1 / output_scale_factor,
and temb acts as a per-channel offset of conv1's output -- the same as
folding its projection into conv1's bias.

UpDecoderBlock2D is checked the same way on the reference test's two cases
(test/src/diffusers/models/unets/unet2d/UpDecoderBlock2D.py: 8 -> 4, two
layers, groups 4 on 1x8x8x8, with and without the upsampler), and an
upsampler conv that passes its centre tap through returns exactly the
nearest 2x repeat of the resnets' output.

Reference modules restated by the functions pinned here:
  resnet_block2d      src/diffusers/models/resnet/ResnetBlock2D.inl:110-195
  up_decoder_block2d  src/diffusers/models/unets/unet2d/UpDecoderBlock2D.cpp:60-74
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import assert_fp32


@pytest.fixture(scope="module")
def vae(orc):
    import oracle.vae as v
    return v


def _params(orc, shapes, seed):
    P = {}
    for i, (name, shape) in enumerate(sorted(shapes.items())):
        mean = 1.0 if name.startswith(("norm1.weight", "norm2.weight")) else 0.0
        P[name] = orc.randn(seed + i, shape, mean=mean, std=0.2)
    return P


def _torch_block(x, P, groups, groups_out, eps, osf, temb):
    """diffusers ResnetBlock2D.forward (pre_norm, SiLU, no dropout) in float64."""
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64))
    x = t(x)
    h = F.silu(F.group_norm(x, groups, t(P["norm1.weight"]), t(P["norm1.bias"]), eps))
    w1 = t(P["conv1.weight"])
    h = F.conv2d(h, w1, t(P["conv1.bias"]), padding=w1.shape[-1] // 2)
    if temb is not None:
        e = F.linear(F.silu(t(temb)), t(P["time_emb_proj.weight"]), t(P["time_emb_proj.bias"]))
        h = h + e[:, :, None, None]
    h = F.silu(F.group_norm(h, groups_out, t(P["norm2.weight"]), t(P["norm2.bias"]), eps))
    w2 = t(P["conv2.weight"])
    h = F.conv2d(h, w2, t(P["conv2.bias"]), padding=w2.shape[-1] // 2)
    if "conv_shortcut.weight" in P:
        b = P.get("conv_shortcut.bias")
        x = F.conv2d(x, t(P["conv_shortcut.weight"]), None if b is None else t(b))
    return ((x + h) / osf).numpy()


CASES = [
    # in, out, temb, groups, groups_out, N, H, W, osf, kernel, shortcut bias
    dict(cin=8, cout=8, temb=None, groups=8, gout=None, N=1, H=2, W=2, osf=1.0, k=3, sb=True),
    dict(cin=8, cout=16, temb=None, groups=8, gout=None, N=1, H=2, W=2, osf=1.0, k=3, sb=True),
    dict(cin=8, cout=8, temb=16, groups=8, gout=None, N=1, H=2, W=2, osf=1.0, k=3, sb=True),
    dict(cin=32, cout=64, temb=24, groups=8, gout=4, N=2, H=6, W=5, osf=2.0, k=3, sb=False),
    dict(cin=16, cout=16, temb=None, groups=4, gout=None, N=1, H=7, W=9, osf=1.5, k=1, sb=True),
]


@pytest.mark.parametrize("c", CASES, ids=lambda c: f"{c['cin']}-{c['cout']}-t{c['temb']}-k{c['k']}")
def test_resnet_block2d_matches_torch(orc, vae, c):
    shapes = vae.resnet_block2d_param_shapes(c["cin"], c["cout"], c["temb"], c["k"],
                                             conv_shortcut_bias=c["sb"])
    assert ("conv_shortcut.weight" in shapes) == (c["cin"] != c["cout"])
    P = _params(orc, shapes, 100)
    x = orc.randn(7, (c["N"], c["cin"], c["H"], c["W"]))
    temb = orc.randn(8, (c["N"], c["temb"])) if c["temb"] else None
    y = vae.resnet_block2d(x, P, c["groups"], c["gout"], 1e-6, c["osf"], temb)
    ref = _torch_block(x, P, c["groups"], c["gout"] or c["groups"], 1e-6, c["osf"], temb)
    assert_fp32(y, ref, tol=2e-5, what="resnet_block2d")


@pytest.mark.parametrize("cout, osf", [(8, 1.0), (8, 3.0), (12, 2.0), (12, 0.7)])
def test_resnet_block2d_zero_conv2_leaves_the_shortcut(orc, vae, cout, osf):
    """conv2 = 0 makes h exactly 0: the block returns shortcut(x) * fl(1 / osf)
    bit for bit (the shortcut an exact 1x1 channel selection plus a bias)."""
    cin = 8
    P = _params(orc, vae.resnet_block2d_param_shapes(cin, cout), 200)
    P["conv2.weight"][:] = 0
    P["conv2.bias"][:] = 0
    x = orc.randn(9, (1, cin, 3, 4))
    r = x
    if cout != cin:
        sel = np.zeros((cout, cin, 1, 1), np.float32)
        for co in range(cout):
            sel[co, co % cin, 0, 0] = 1.0
        P["conv_shortcut.weight"] = sel
        r = (x[:, [co % cin for co in range(cout)]] + P["conv_shortcut.bias"][None, :, None, None]).astype(np.float32)
    y = vae.resnet_block2d(x, P, 4, None, 1e-6, osf)
    want = (r * (np.float32(1.0) / np.float32(osf))).astype(np.float32)
    assert np.array_equal(y, want)


def test_resnet_block2d_temb_is_conv1_bias_offset(orc, vae):
    """The projected SiLU(temb) is added per (sample, channel) to conv1's
    output: folding it into conv1's bias gives the same block (to fp32
    rounding), while a temb that skipped the SiLU would not."""
    cin, cout, tc = 8, 16, 12
    P = _params(orc, vae.resnet_block2d_param_shapes(cin, cout, tc), 300)
    x = orc.randn(10, (1, cin, 4, 4))
    temb = orc.randn(11, (1, tc), std=2.0)
    y = vae.resnet_block2d(x, P, 4, None, 1e-6, 1.0, temb)
    silu = temb / (1.0 + np.exp(-temb.astype(np.float64)))
    off = silu @ P["time_emb_proj.weight"].astype(np.float64).T + P["time_emb_proj.bias"]
    Q = dict(P)
    del Q["time_emb_proj.weight"], Q["time_emb_proj.bias"]
    Q["conv1.bias"] = (P["conv1.bias"] + off[0]).astype(np.float32)
    assert_fp32(y, vae.resnet_block2d(x, Q, 4, None, 1e-6, 1.0), tol=2e-5, what="temb as a bias")
    raw = temb @ P["time_emb_proj.weight"].astype(np.float64).T + P["time_emb_proj.bias"]
    Q["conv1.bias"] = (P["conv1.bias"] + raw[0]).astype(np.float32)
    assert not np.allclose(y, vae.resnet_block2d(x, Q, 4, None, 1e-6, 1.0), atol=1e-3)


def test_resnet_block2d_temb_vanishes_under_per_channel_groups(orc, vae):
    """With one channel per norm2 group, a per-channel offset is removed by
    the mean subtraction: the block ignores temb (to fp32 rounding)."""
    cin, cout, tc = 8, 8, 6
    P = _params(orc, vae.resnet_block2d_param_shapes(cin, cout, tc), 400)
    x = orc.randn(12, (1, cin, 5, 5))
    temb = orc.randn(13, (1, tc))
    a = vae.resnet_block2d(x, P, 4, cout, 1e-6, 1.0, temb)
    b = vae.resnet_block2d(x, P, 4, cout, 1e-6, 1.0, None)
    assert_fp32(a, b, tol=1e-4, what="per-channel groups")
    c = vae.resnet_block2d(x, P, 4, 2, 1e-6, 1.0, temb)
    d = vae.resnet_block2d(x, P, 4, 2, 1e-6, 1.0, None)
    assert not np.allclose(c, d, atol=1e-3)


@pytest.mark.parametrize("add_upsample", [False, True])
def test_up_decoder_block2d_matches_torch(orc, vae, add_upsample):
    shapes = vae.up_decoder_block2d_param_shapes(8, 4, 2, add_upsample)
    P = _params(orc, shapes, 500)
    x = orc.randn(14, (1, 8, 8, 8))
    y = vae.up_decoder_block2d(x, P, 2, 4, 1e-6, 1.0, add_upsample)
    h = x
    for i in range(2):
        sub = {k[len(f"resnets.{i}."):]: v for k, v in P.items() if k.startswith(f"resnets.{i}.")}
        h = _torch_block(h, sub, 4, 4, 1e-6, 1.0, None)
    if add_upsample:
        t = torch.from_numpy(np.asarray(h, np.float64))
        t = F.interpolate(t, scale_factor=2, mode="nearest")
        w = torch.from_numpy(P["upsamplers.0.conv.weight"].astype(np.float64))
        b = torch.from_numpy(P["upsamplers.0.conv.bias"].astype(np.float64))
        h = F.conv2d(t, w, b, padding=1).numpy()
    assert y.shape == ((1, 4, 16, 16) if add_upsample else (1, 4, 8, 8))
    assert_fp32(y, h, tol=2e-5, what="up_decoder_block2d")


def test_up_decoder_block2d_centre_tap_upsampler_repeats_pixels(orc, vae):
    P = _params(orc, vae.up_decoder_block2d_param_shapes(8, 4, 1, True), 600)
    w = np.zeros((4, 4, 3, 3), np.float32)
    for c in range(4):
        w[c, c, 1, 1] = 1.0
    P["upsamplers.0.conv.weight"] = w
    P["upsamplers.0.conv.bias"] = np.zeros(4, np.float32)
    x = orc.randn(15, (1, 8, 5, 7))
    y = vae.up_decoder_block2d(x, P, 1, 4, 1e-6, 1.0, True)
    h = vae.up_decoder_block2d(x, P, 1, 4, 1e-6, 1.0, False)
    assert np.array_equal(y, np.repeat(np.repeat(h, 2, axis=2), 2, axis=3))
