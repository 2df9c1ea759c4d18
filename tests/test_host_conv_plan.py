"""Planning of the VAE decoder's convolution nodes without a device
(dt_graph_plan on host descriptors): Conv2d::forward's ADD(CONV_2D_DIRECT,
bias[1, Co, 1, 1]) (src/nn/modules/conv/Conv2d.cpp:38-102) becomes one
convolution with the bias in its epilogue, and Upsample2D's nearest 2x
UPSCALE (src/diffusers/models/resnet/Upsample2D.cpp:50-72) folds into the
conv's input when the conv is its only consumer."""
import os
import re

import torch

import dit_hip as dh
from conftest import ROOT
from graphkit import Graph


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
