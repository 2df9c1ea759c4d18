"""Planning of the VAE decoder's convolution nodes without a device
(dt_graph_plan on host descriptors): Conv2d::forward's ADD(CONV_2D_DIRECT,
bias[1, Co, 1, 1]) (src/nn/modules/conv/Conv2d.cpp:38-102) becomes one
convolution with the bias in its epilogue, and Upsample2D's nearest 2x
UPSCALE (src/diffusers/models/resnet/Upsample2D.cpp:50-72) folds into the
conv's input when the conv is its only consumer.  ResnetBlock2D's tail,
`(input + hidden) / output_scale_factor` (src/diffusers/models/resnet/
ResnetBlock2D.inl:194: ADD(res, conv2) then SCALE), folds into conv2's
epilogue when conv2's output and the ADD are used nowhere else; the memory
replay lets the output sit exactly on the residual but not on the conv's
input.  A GroupNorm (+ affine) (+ SiLU) chain read only by a 3x3 conv
(ResnetBlock2D.inl:114-127, 163-176) is applied in the conv's channel-last
copy."""
import os
import re

import torch

import dit_hip as dh
from conftest import ROOT
from graphkit import Graph, fbits


def _conv_graph(up=None, bias=True, Ci=8, Co=16, K=3, H=6, W=10):
    g = Graph(device="cpu")
    x = g.leaf(torch.zeros((1, Ci, H, W)))
    w = g.leaf(torch.zeros((Co, Ci, K, K)))
    b = g.leaf(torch.zeros((Co,)))
    u = g.upscale(x, up) if up else x
    c = g.conv_2d_direct(w, u, p0=(K - 1) // 2, p1=(K - 1) // 2)
    y = g.add(c, g.reshape(b, [1, 1, Co, 1])) if bias else c
    return g, u, c, y


def _index(g, node):
    return next(i for i, n in enumerate(g.nodes) if n is node)


def test_bias_add_and_upscale_fold_into_the_conv():
    g, u, c, y = _conv_graph(up=2)
    roots = g.plan(outputs=[y])
    iy = _index(g, y)
    assert roots[_index(g, c)] == iy and roots[_index(g, u)] == iy
    assert roots[iy] == -1
    assert sum(r >= 0 for r in roots) == 2   # the bias VIEW runs as a view
    assert c.ne == [20, 12, 16, 1]


def test_conv_without_bias_or_upscale_runs_alone():
    g, u, c, y = _conv_graph(bias=False)
    assert g.plan(outputs=[y]) == [-1] * len(g.nodes)


def test_upscale_not_folded_when_it_is_an_output_or_not_2x():
    g, u, c, y = _conv_graph(up=2)
    roots = g.plan(outputs=[y, u])          # the upsampled tensor is wanted
    assert roots[_index(g, u)] == -1 and roots[_index(g, c)] == _index(g, y)
    g, u, c, y = _conv_graph(up=3)
    roots = g.plan(outputs=[y])
    assert roots[_index(g, u)] == -1 and roots[_index(g, c)] == _index(g, y)


def test_conv_kept_when_its_output_is_wanted():
    g, u, c, y = _conv_graph(up=2, K=1)
    roots = g.plan(outputs=[y, c])
    # the bias ADD runs on its own; the conv still reads the upscale on the fly
    assert roots[_index(g, y)] == -1 and roots[_index(g, c)] == -1
    assert roots[_index(g, u)] == _index(g, c)


def test_op_ids_follow_the_header():
    text = open(os.path.join(ROOT, "include", "dit_hip.h")).read()
    body = text[text.index("DT_OP_NONE = 0"):text.index("DT_OP_COUNT")]
    code = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    names = re.findall(r"DT_OP_(\w+)", code)
    assert names.index("CONV_2D_DIRECT") == dh.OP_CONV_2D_DIRECT
    assert names.index("UPSCALE") == dh.OP_UPSCALE
    assert names.index("MUL_MAT") == dh.OP_MUL_MAT and names.index("UNARY") == dh.OP_UNARY


def _resnet_tail(Ci=8, Co=16, K=3, H=6, W=10, scale=0.5, res_type=torch.float32, res_shape=None):
    """x -> conv(+bias) = h; y = SCALE(ADD(res, h), scale)."""
    g = Graph(device="cpu")
    x = g.leaf(torch.zeros((1, Ci, H, W)))
    w = g.leaf(torch.zeros((Co, Ci, K, K)))
    b = g.leaf(torch.zeros((Co,)))
    r = g.leaf(torch.zeros(res_shape or (1, Co, H, W), dtype=res_type))
    c = g.conv_2d_direct(w, x, p0=(K - 1) // 2, p1=(K - 1) // 2)
    h = g.add(c, g.reshape(b, [1, 1, Co, 1]))
    s = g.add(h, r) if res_shape else g.add(r, h)
    y = g.scale(s, scale)
    return g, x, r, c, h, s, y


def test_residual_add_and_scale_fold_into_the_conv():
    g, x, r, c, h, s, y = _resnet_tail()
    roots = g.plan(outputs=[y])
    iy = _index(g, y)
    assert [roots[_index(g, t)] for t in (c, h, s)] == [iy] * 3 and roots[iy] == -1


def test_residual_add_folds_alone_when_the_sum_is_wanted():
    g, x, r, c, h, s, y = _resnet_tail()
    roots = g.plan(outputs=[y, s])
    i_s = _index(g, s)
    assert roots[_index(g, c)] == i_s and roots[_index(g, h)] == i_s
    assert roots[i_s] == -1 and roots[_index(g, y)] == -1
    # a SCALE with a bias term (ggml_scale_bias) is not the module's division: the ADD folds alone
    g, x, r, c, h, s, y = _resnet_tail()
    y.d.op_params[1] = fbits(0.25)
    roots = g.plan(outputs=[y])
    assert roots[_index(g, h)] == _index(g, s) and roots[_index(g, y)] == -1


def test_residual_not_folded_when_the_conv_output_is_wanted_or_does_not_match():
    g, x, r, c, h, s, y = _resnet_tail()
    roots = g.plan(outputs=[y, h])
    assert roots[_index(g, c)] == _index(g, h)
    assert roots[_index(g, s)] == -1 and roots[_index(g, y)] == -1
    # a residual of another type, or one broadcast over the image, stays an ADD of its own
    for kw in (dict(res_type=torch.bfloat16), dict(res_shape=(1, 16, 1, 1))):
        g, x, r, c, h, s, y = _resnet_tail(**kw)
        roots = g.plan(outputs=[y])
        assert roots[_index(g, c)] == _index(g, h), kw
        assert roots[_index(g, s)] == -1 and roots[_index(g, y)] == -1, kw


def test_residual_fold_may_write_over_the_residual_only():
    # the output exactly on the residual: each element is read by the lane that writes it
    g, x, r, c, h, s, y = _resnet_tail()
    y.d.data = r.d.data
    roots, runs, held = g.plan_checked(outputs=[y])
    assert roots[_index(g, s)] == _index(g, y) and held == 0
    # partly over the residual, or over the conv's input (read by every tile): not fused there
    for target, off in (("res", 128), ("input", 0)):
        g, x, r, c, h, s, y = _resnet_tail()
        y.d.data = (r if target == "res" else x).d.data + off
        roots, runs, held = g.plan_checked(outputs=[y])
        assert roots[_index(g, s)] != _index(g, y) and held >= 1, (off, roots)


def _gn_conv(K=3, affine=True, silu=True, up=False, C=16, G=4, Co=8, H=6, W=10):
    """GroupNorm::forward (reshape, NORM, reshape, MUL w, ADD b) + SiLU, then a conv + bias."""
    g = Graph(device="cpu")
    x = g.leaf(torch.zeros((1, C, H, W)))
    v = g.reshape(x, [C // G * H * W, G, 1])
    n = g.norm(v, 1e-6)
    cur = g.reshape(n, [W, H, C, 1])
    if affine:
        cur = g.mul(cur, g.reshape(g.leaf(torch.zeros((C,))), [1, 1, C, 1]))
        cur = g.add(cur, g.reshape(g.leaf(torch.zeros((C,))), [1, 1, C, 1]))
    if silu:
        cur = g.mul(cur, g.sigmoid(cur))
    gn = cur
    u = g.upscale(gn, 2) if up else gn
    w = g.leaf(torch.zeros((Co, C, K, K)))
    b = g.leaf(torch.zeros((Co,)))
    c = g.conv_2d_direct(w, u, p0=(K - 1) // 2, p1=(K - 1) // 2)
    y = g.add(c, g.reshape(b, [1, 1, Co, 1]))
    return g, n, gn, c, y


def test_groupnorm_folds_into_the_3x3_conv_copy():
    for kw in (dict(), dict(affine=False), dict(silu=False), dict(up=True)):
        g, n, gn, c, y = _gn_conv(**kw)
        roots = g.plan(outputs=[y])
        iy = _index(g, y)
        assert roots[_index(g, n)] == iy and roots[_index(g, gn)] == iy and roots[_index(g, c)] == iy, kw
        assert roots[iy] == -1, kw


def test_groupnorm_not_folded_into_1x1_convs_or_when_wanted():
    g, n, gn, c, y = _gn_conv(K=1)
    roots = g.plan(outputs=[y])
    assert roots[_index(g, n)] == _index(g, gn) and roots[_index(g, gn)] == -1
    g, n, gn, c, y = _gn_conv()
    roots = g.plan(outputs=[y, gn])
    assert roots[_index(g, n)] == _index(g, gn) and roots[_index(g, gn)] == -1
    assert roots[_index(g, c)] == _index(g, y)
    # a bare NORM (no affine, no SiLU) is not a GroupNorm chain
    g, n, gn, c, y = _gn_conv(affine=False, silu=False)
    roots = g.plan(outputs=[y])
    assert roots[_index(g, n)] == -1


def test_residual_goes_to_the_3x3_conv_when_both_operands_are_convs():
    """A block with a 1x1 conv_shortcut adds two conv outputs: the 3x3 conv2
    takes the residual (its epilogue stages through LDS), whichever ADD
    operand it is; the shortcut stays a conv of its own."""
    for swap in (False, True):
        g = Graph(device="cpu")
        x = g.leaf(torch.zeros((1, 8, 6, 10)))
        hin = g.leaf(torch.zeros((1, 16, 6, 10)))
        ws, bs = g.leaf(torch.zeros((16, 8, 1, 1))), g.leaf(torch.zeros((16,)))
        w3, b3 = g.leaf(torch.zeros((16, 16, 3, 3))), g.leaf(torch.zeros((16,)))
        sc = g.add(g.conv_2d_direct(ws, x, p0=0, p1=0), g.reshape(bs, [1, 1, 16, 1]))
        c3 = g.conv_2d_direct(w3, hin, p0=1, p1=1)
        h = g.add(c3, g.reshape(b3, [1, 1, 16, 1]))
        s = g.add(h, sc) if swap else g.add(sc, h)
        y = g.scale(s, 1.0)
        roots = g.plan(outputs=[y])
        iy = _index(g, y)
        assert [roots[_index(g, t)] for t in (c3, h, s)] == [iy] * 3, swap
        assert roots[_index(g, sc)] == -1, swap
