"""GPU parity of the unfused ggml-op kernels and of dt_graph_compute.

Graphs are emitted node for node as the reference's modules emit them
through Runtime (LayerNorm + modulation, RMSNorm + Flux2PosEmbed with its
per-axis views, position-column CONTs and left-nested CONCATs, SwiGLU as
SIGMOID/MUL/MUL, gated residual, GroupNorm's reshape/NORM/reshape/MUL/ADD +
SiLU), then executed by the library.  Each output is checked against the
oracle; the fusion statistics confirm which path ran."""
import ctypes

import numpy as np
import pytest
import torch

import dit_hip as dh
from conftest import assert_bf16, assert_fp32
from graphkit import Backend, Graph
from test_gpu_fused import as_input, check, dev_tensor, flux_positions, host

pytestmark = pytest.mark.gpu

SEED = 0x5EED1000
DT = [torch.bfloat16, torch.float32]
TY = {torch.bfloat16: dh.BF16, torch.float32: dh.F32}


@pytest.fixture
def be(dev):
    b = Backend()
    yield b.h
    torch.cuda.synchronize()
    b.close()


# ------------------------------------------------------------ unfused ops ----
@pytest.mark.parametrize("dtype", DT)
def test_binary_broadcast(orc, dev, dtype):
    a = orc.randn(SEED, (2, 3, 4, 8))
    for bshape in [(8,), (1, 3, 1, 8), (2, 1, 4, 1), (1, 1, 2, 4)]:
        b = orc.randn(SEED + 1, bshape)
        for op in range(4):
            ad = dev_tensor(a, dtype)
            bd = dev_tensor(b, torch.float32)       # mixed operand types
            out = torch.empty_like(ad)
            dh.op_binary(op, ad, bd, out)
            torch.cuda.synchronize()
            check(host(out), orc.binary(op, as_input(a, dtype), b), dtype, f"binary{op}{bshape}")


def test_binary_strided_src(orc, dev):
    a = orc.randn(SEED + 2, (6, 10))
    ad = dev_tensor(a, torch.float32).t()          # [10, 6] transposed view
    b = orc.randn(SEED + 3, (6,))
    out = torch.empty((10, 6), device="cuda")
    dh.op_binary(dh.BIN_MUL, ad, dev_tensor(b, torch.float32), out)
    torch.cuda.synchronize()
    assert_fp32(host(out), orc.binary(2, a.T, b), what="strided")


@pytest.mark.parametrize("dtype", DT)
def test_unary(orc, dev, dtype):
    x = as_input(orc.randn(SEED + 4, (5, 37)) * 3, dtype)       # values the device sees
    xa = as_input(np.abs(x) + 0.5, dtype)
    f64 = lambda a: a.astype(np.float64)
    cases = [(dh.UN_SIGMOID, x, orc.sigmoid(x), 0, 0),
             (dh.UN_SCALE, x, x * np.float32(0.375), 0.375, 0),
             (dh.UN_CLAMP, x, np.clip(x, -1.0, 2.0), -1.0, 2.0),
             (dh.UN_EXP, x, np.exp(f64(x)), 0, 0),
             (dh.UN_SQRT, xa, np.sqrt(f64(xa)), 0, 0),
             (dh.UN_LOG, xa, np.log(f64(xa)), 0, 0),
             (dh.UN_SIN, x, np.sin(f64(x)), 0, 0),
             (dh.UN_COS, x, np.cos(f64(x)), 0, 0),
             (dh.UN_SILU, x, f64(x) / (1 + np.exp(-f64(x))), 0, 0)]
    for op, inp, want, p0, p1 in cases:
        src = dev_tensor(inp, dtype)
        out = torch.empty_like(src)
        dh.op_unary(op, src, out, p0, p1)
        torch.cuda.synchronize()
        check(host(out), want, dtype, f"unary{op}")
    out = torch.empty((3, 4), dtype=dtype, device="cuda")
    dh.op_unary(dh.UN_FILL, None, out, 1.5)
    assert np.all(host(out) == 1.5)


@pytest.mark.parametrize("dtype", DT)
def test_norm_rms_norm_strided_rows(orc, dev, dtype):
    big = orc.randn(SEED + 5, (7, 300))
    d = dev_tensor(big, dtype)
    v = d[:, 20:276]                                # 256-wide rows, row stride 300
    for rms in (False, True):
        out = torch.empty((7, 256), dtype=dtype, device="cuda")
        dh.op_norm(v, out, 1e-6, rms=rms)
        torch.cuda.synchronize()
        x = as_input(big[:, 20:276], dtype)
        want = orc.rms_norm(x, 1e-6) if rms else orc.norm(x, 1e-6)
        check(host(out), want, dtype, "rms" if rms else "norm")


@pytest.mark.parametrize("dtype", DT)
def test_rope_ext_on_axis_view(orc, dev, dtype):
    # one Flux2PosEmbed section: x[..., 64:96] of [1, S, H, 128], n_dims 32
    pos = flux_positions(16, 4)
    S = pos.shape[0]
    x = orc.randn(SEED + 6, (1, S, 3, 128))
    xd = dev_tensor(x, dtype)
    view = xd[..., 64:96]
    out = torch.empty((1, S, 3, 32), dtype=dtype, device="cuda")
    p = torch.from_numpy(np.ascontiguousarray(pos[:, 2])).cuda()
    dh.op_rope(view, p, out, 32, 2000.0)
    torch.cuda.synchronize()
    want = orc.rope_normal(as_input(x, dtype)[..., 64:96], pos[:, 2], 32, 2000.0)
    check(host(out), want, dtype, "rope")
    # n_dims < ne0: the tail passes through
    out2 = torch.empty_like(out)
    dh.op_rope(view, p, out2, 16, 2000.0)
    torch.cuda.synchronize()
    check(host(out2), orc.rope_normal(as_input(x, dtype)[..., 64:96], pos[:, 2], 16, 2000.0), dtype, "rope16")


def test_concat_and_cpy(orc, dev):
    a = orc.randn(SEED + 7, (2, 3, 4, 5))
    b = orc.randn(SEED + 8, (2, 3, 4, 5))
    for dim in range(4):
        axis = 3 - dim
        bb = b.take(range(2 if b.shape[axis] > 2 else 1), axis=axis)
        out_shape = list(a.shape)
        out_shape[axis] += bb.shape[axis]
        out = torch.empty(out_shape, device="cuda")
        dh.op_concat(dev_tensor(a, torch.float32), dev_tensor(np.ascontiguousarray(bb), torch.float32), dim, out)
        torch.cuda.synchronize()
        assert np.array_equal(host(out), np.concatenate([a, bb], axis=axis))
    # transposed f32 -> contiguous bf16
    t = dev_tensor(a, torch.float32).permute(0, 2, 1, 3)
    o = torch.empty(t.shape, dtype=torch.bfloat16, device="cuda")
    dh.op_cpy(t, o)
    torch.cuda.synchronize()
    assert np.array_equal(host(o), orc.round_bf16(np.ascontiguousarray(a.transpose(0, 2, 1, 3))))
    # I32 raw copy of a strided column and I32 concat
    pos = torch.from_numpy(flux_positions(8, 4)).cuda()
    col = torch.empty(pos.shape[0], dtype=torch.int32, device="cuda")
    dh.op_cpy(pos[:, 3], col)
    cat = torch.empty((2 * pos.shape[0], 4), dtype=torch.int32, device="cuda")
    dh.op_concat(pos, pos, 1, cat)
    torch.cuda.synchronize()
    assert torch.equal(col, pos[:, 3]) and torch.equal(cat, torch.cat([pos, pos]))
    # dense bf16 runs of whole 16-byte vectors (the txt | img token concat of
    # the single-stream input): the vector-copy path, bit for bit
    t_ = dev_tensor(orc.randn(SEED + 9, (1, 512, 3072)), torch.bfloat16)
    i_ = dev_tensor(orc.randn(SEED + 10, (1, 4096, 3072)), torch.bfloat16)
    j = torch.empty((1, 4608, 3072), dtype=torch.bfloat16, device="cuda")
    dh.op_concat(t_, i_, 1, j)
    torch.cuda.synchronize()
    assert torch.equal(j, torch.cat([t_, i_], 1))


# ------------------------------------------------------------------ graphs ----
def seq_positions(n_txt, n_img, width=8):
    txt = [[0, 0, 0, l] for l in range(n_txt)]
    img = [[0, i // width, i % width, 0] for i in range(n_img)]
    return np.array(txt + img, dtype=np.int32).reshape(-1, 4)


def pos_columns(g, pos_leaf, S):
    """position_ids[:, a] as the reference emits it: narrow (view), CONT
    (the view is not contiguous), reshape to a vector."""
    cols = []
    for a in range(4):
        v = g.view(pos_leaf, [1, S], [4, 16], 4 * a)
        c = g.cont(v)
        cols.append(g.reshape(c, [S]))
    return cols


def emit_qk(g, q_leaf, w_leaf, pos_cols, axis_dim, theta, es):
    """RMSNorm(q) * w, then 4x rope_ext on the axis views and the
    left-nested pairwise concat (Tensor::cat)."""
    rn = g.rms_norm(q_leaf, 1e-6)
    wm = g.mul(rn, w_leaf)
    return emit_rope(g, wm, pos_cols, axis_dim, theta, es)


def emit_rope(g, x, pos_cols, axis_dim, theta, es):
    ne = x.ne
    nb = list(x.d.nb)
    secs = []
    for a, pc in enumerate(pos_cols):
        v = g.view(x, [axis_dim] + ne[1:], nb, a * axis_dim * es)
        secs.append(g.rope_ext(v, pc, axis_dim, 0, theta))
    out = secs[0]
    for s in secs[1:]:
        out = g.concat(out, s, 0)
    return out


def build_single_block_chain(orc, dtype, S, D, H, I, theta=2000.0):
    es = 2 if dtype == torch.bfloat16 else 4
    g = Graph()
    raw = {
        "x": orc.randn(SEED + 10, (1, S, D)), "mod": orc.randn(SEED + 11, (1, 1, 3 * D), std=0.1),
        "q": orc.randn(SEED + 12, (1, S, H, 128)), "k": orc.randn(SEED + 13, (1, S, H, 128)),
        "wq": orc.randn(SEED + 14, (128,), mean=1.0, std=0.02),
        "wk": orc.randn(SEED + 15, (128,), mean=1.0, std=0.02),
        "g": orc.randn(SEED + 16, (1, S, I)), "u": orc.randn(SEED + 17, (1, S, I)),
        "o": orc.randn(SEED + 18, (1, S, D)),
    }
    pos = seq_positions(S // 3, S - S // 3)
    L = {k: g.leaf(dev_tensor(v, torch.float32 if k in ("mod", "wq", "wk") else dtype))
         for k, v in raw.items()}
    L["pos"] = g.leaf(torch.from_numpy(pos).cuda())
    # modulation chunks: shift, scale, gate views of the [1,1,3D] output
    shift = g.view(L["mod"], [D, 1, 1], [4, 4 * 3 * D, 4 * 3 * D], 0)
    scale = g.view(L["mod"], [D, 1, 1], [4, 4 * 3 * D, 4 * 3 * D], 4 * D)
    gate = g.view(L["mod"], [D, 1, 1], [4, 4 * 3 * D, 4 * 3 * D], 8 * D)
    one = g.fill([1], dh.F32, 1.0)
    t = g.add(scale, one)                                   # 1.0f + scale
    n = g.norm(L["x"], 1e-6)
    m = g.mul(n, t)
    ada = g.add(m, shift)
    cols = pos_columns(g, L["pos"], S)
    qr = emit_qk(g, L["q"], L["wq"], cols, 32, theta, es)
    kr = emit_qk(g, L["k"], L["wk"], cols, 32, theta, es)
    sg = g.sigmoid(L["g"])
    silu = g.mul(L["g"], sg)
    sw = g.mul(silu, L["u"])
    go = g.mul(L["o"], gate)
    res = g.add(L["x"], go)
    outs = {"adaln": ada, "q": qr, "k": kr, "swiglu": sw, "residual": res}
    return g, raw, pos, outs, {"n": n, "t": t}


def oracle_single_block(orc, raw, pos, dtype, D, theta):
    r = {k: (as_input(v, dtype) if k not in ("mod", "wq", "wk") else v) for k, v in raw.items()}
    mod = r["mod"].reshape(-1)
    shift, scale, gate = mod[:D], mod[D:2 * D], mod[2 * D:]
    return {
        "adaln": orc.adaln(r["x"][0], shift, scale, 1e-6),
        "q": orc.qk_rmsnorm_rope(r["q"][0], r["wq"], pos, 32, theta, 1e-6),
        "k": orc.qk_rmsnorm_rope(r["k"][0], r["wk"], pos, 32, theta, 1e-6),
        "swiglu": orc.swiglu(r["g"][0], r["u"][0]),
        "residual": orc.gated_residual(r["x"][0], r["o"][0], gate),
    }


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("S,D,H,I", [(48, 3072, 24, 9216), (12, 256, 2, 512)])
def test_graph_single_block_chain_fused(orc, be, dtype, S, D, H, I):
    g, raw, pos, outs, _ = build_single_block_chain(orc, dtype, S, D, H, I)
    roots = g.plan(outputs=outs.values())
    kernels, fused = g.compute(be, outputs=outs.values())
    assert sum(r >= 0 for r in roots) == fused
    # every absorbed node is absorbed by a later node that runs a fused kernel
    assert all(r > i and roots[r] == -1 for i, r in enumerate(roots) if r >= 0)
    torch.cuda.synchronize()
    want = oracle_single_block(orc, raw, pos, dtype, D, 2000.0)
    for name, node in outs.items():
        got = host(node.torch()).reshape(want[name].shape)
        check(got, want[name], dtype, name)
    # adaLN with its 1 + scale + 4 position CONTs + (q, k and SwiGLU in one
    # launch) + residual
    assert kernels == 7, kernels
    # claimed nodes: norm + mul and the fill + (scale+1) of the factor (4);
    # per q/k: rms, mul, 4 views, 4 ropes and the 2 inner concats (12 each);
    # swiglu sigmoid + mul (2); residual mul (1)
    assert fused == 4 + 24 + 2 + 1, fused


@pytest.mark.parametrize("dtype", DT)
def test_graph_scale_factor_kept_when_it_is_an_output(orc, be, dtype):
    """The adaLN absorbs the FILL + ADD of its 1 + scale only when nothing
    else reads that factor: with the factor requested as an output, its ADD
    and FILL run as their own kernels (2 more launches, 2 fewer absorbed
    nodes), the adaLN reads the stored factor, and every output -- the
    factor included -- still matches the oracle."""
    S, D, H, I = 12, 256, 2, 512
    g, raw, pos, outs, inner = build_single_block_chain(orc, dtype, S, D, H, I)
    kernels, fused = g.compute(be, outputs=list(outs.values()) + [inner["t"]])
    torch.cuda.synchronize()
    want = oracle_single_block(orc, raw, pos, dtype, D, 2000.0)
    for name, node in outs.items():
        check(host(node.torch()).reshape(want[name].shape), want[name], dtype, name)
    scale = raw["mod"].reshape(-1)[D:2 * D]
    assert np.array_equal(host(inner["t"].torch()).reshape(D), (scale + np.float32(1.0)).astype(np.float32))
    assert kernels == 7 + 2 and fused == 4 + 24 + 2 + 1 - 2, (kernels, fused)


@pytest.mark.parametrize("dtype", DT)
def test_graph_unfused_when_intermediates_are_outputs(orc, be, dtype):
    S, D, H, I = 12, 256, 2, 512
    g, raw, pos, outs, inner = build_single_block_chain(orc, dtype, S, D, H, I)
    # Asking for the LayerNorm output forces NORM/MUL/ADD to run one by one.
    kernels, fused = g.compute(be, outputs=list(outs.values()) + [inner["n"]])
    torch.cuda.synchronize()
    want = oracle_single_block(orc, raw, pos, dtype, D, 2000.0)
    for name, node in outs.items():
        # unfused adaLN rounds NORM, MUL and ADD outputs to the node type
        check(host(node.torch()).reshape(want[name].shape), want[name], dtype, name,
              one_rounding=name != "adaln")
    check(host(inner["n"].torch()).reshape(S, D), orc.norm(as_input(raw["x"], dtype)[0], 1e-6), dtype,
          "norm")
    assert kernels == 11 and fused == 24 + 2 + 1, (kernels, fused)


@pytest.mark.parametrize("dtype", DT)
def test_graph_double_stream_qk_concat(orc, be, dtype):
    # Flux2Attention: txt and img q normalised with their own weights,
    # cat(txt, img) along the sequence, then Flux2PosEmbed on the joint q.
    St, Si, H = 8, 16, 3
    es = 2 if dtype == torch.bfloat16 else 4
    g = Graph()
    qt, qi = orc.randn(SEED + 20, (1, St, H, 128)), orc.randn(SEED + 21, (1, Si, H, 128))
    wt = orc.randn(SEED + 22, (128,), mean=1.0, std=0.02)
    wi = orc.randn(SEED + 23, (128,), mean=1.0, std=0.02)
    pos = flux_positions(St, 4)
    Lt, Li = g.leaf(dev_tensor(qt, dtype)), g.leaf(dev_tensor(qi, dtype))
    Wt, Wi = g.leaf(dev_tensor(wt, torch.float32)), g.leaf(dev_tensor(wi, torch.float32))
    P = g.leaf(torch.from_numpy(pos).cuda())
    zt = g.mul(g.rms_norm(Lt, 1e-6), Wt)
    zi = g.mul(g.rms_norm(Li, 1e-6), Wi)
    z = g.concat(zt, zi, 2)
    out = emit_rope(g, z, pos_columns(g, P, St + Si), 32, 10000.0, es)
    kernels, fused = g.compute(be, outputs=[out])
    torch.cuda.synchronize()
    x = np.concatenate([as_input(qt, dtype)[0], as_input(qi, dtype)[0]])
    # the two segments use different weights: run the oracle per segment
    want = np.concatenate([
        orc.qk_rmsnorm_rope(x[:St], wt, pos[:St], 32, 10000.0, 1e-6),
        orc.qk_rmsnorm_rope(x[St:], wi, pos[St:], 32, 10000.0, 1e-6)])
    check(host(out.torch())[0], want, dtype, "double-stream q")
    assert kernels == 4 + 2, kernels     # 4 position CONTs + one fused launch per segment


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("affine,silu", [(True, True), (True, False), (False, True)])
def test_graph_groupnorm_silu(orc, be, dtype, affine, silu):
    N, C, Hh, W, G = 1, 64, 16, 16, 32
    g = Graph()
    x = orc.randn(SEED + 30, (N, C, Hh, W))
    w = orc.randn(SEED + 31, (C,), mean=1.0, std=0.02)
    b = orc.randn(SEED + 32, (C,), std=0.02)
    X = g.leaf(dev_tensor(x, dtype))
    v = g.reshape(X, [C // G * Hh * W, G, N])
    n = g.norm(v, 1e-6)
    r = g.reshape(n, [W, Hh, C, N])
    cur = r
    if affine:
        cur = g.mul(cur, g.leaf(dev_tensor(w.reshape(1, C, 1, 1), torch.float32)))
        cur = g.add(cur, g.leaf(dev_tensor(b.reshape(1, C, 1, 1), torch.float32)))
    if silu:
        cur = g.mul(cur, g.sigmoid(cur))
    kernels, fused = g.compute(be, outputs=[cur])
    torch.cuda.synchronize()
    want = orc.groupnorm_silu(as_input(x, dtype), G, w if affine else None, b if affine else None,
                              1e-6, silu=silu)
    check(host(cur.torch()), want, dtype, "gn graph")
    assert kernels == 2, kernels          # stats + apply


@pytest.mark.parametrize("segments", [1, 2])
def test_graph_attention_takes_the_q_chain(orc, be, segments):
    """FLASH_ATTN_EXT on the permuted QK-RMSNorm+RoPE root (one segment, or
    txt | img with their own weights as in Flux2Attention.hpp:93-116): the
    chain becomes the attention's prologue -- one launch instead of one per
    segment plus the attention -- and the output is bit-identical to the
    graph that keeps q (the root flagged as an output)."""
    n_txt, n_img, H = (0, 200, 3) if segments == 1 else (24, 136, 2)
    S = n_txt + n_img
    pos = seq_positions(n_txt, n_img, 16)
    raw = {"q": orc.randn(SEED + 60, (1, S, H, 128)), "k": orc.randn(SEED + 61, (1, S, H, 128)),
           "v": orc.randn(SEED + 62, (1, S, H, 128)),
           "w0": orc.randn(SEED + 63, (128,), mean=1.0, std=0.1), "w1": orc.randn(SEED + 64, (128,), mean=1.0, std=0.1)}
    outs = []
    for keep_q in (False, True):
        g = Graph()
        L = {k: g.leaf(dev_tensor(v, torch.float32 if k[0] == "w" else torch.bfloat16)) for k, v in raw.items()}
        P = g.leaf(torch.from_numpy(pos).cuda())
        if segments == 1:
            y = emit_qk(g, L["q"], L["w0"], pos_columns(g, P, S), 32, 10000.0, 2)
        else:
            qt = g.leaf(dev_tensor(raw["q"][:, :n_txt], torch.bfloat16))
            qi = g.leaf(dev_tensor(raw["q"][:, n_txt:], torch.bfloat16))
            z = g.concat(g.mul(g.rms_norm(qt, 1e-6), L["w0"]), g.mul(g.rms_norm(qi, 1e-6), L["w1"]), 2)
            y = emit_rope(g, z, pos_columns(g, P, S), 32, 10000.0, 2)
        o = g.flash_attn_ext(g.permute_tokens_heads(y), g.permute_tokens_heads(L["k"]),
                             g.permute_tokens_heads(L["v"]), 1.0 / 128 ** 0.5)
        kernels, fused = g.compute(be, outputs=[o, y] if keep_q else [o])
        torch.cuda.synchronize()
        # 4 position CONTs + the attention (+ one QK launch per segment when q is kept)
        assert kernels == 5 + (segments if keep_q else 0), (keep_q, kernels)
        outs.append(o.torch().clone())
    assert torch.equal(outs[0], outs[1])
    x = as_input(raw["q"], torch.bfloat16)[0]
    segs = [(0, n_txt, raw["w0"]), (n_txt, S, raw["w1"])] if segments == 2 else [(0, S, raw["w0"])]
    qn = np.concatenate([orc.qk_rmsnorm_rope(x[a:b], w, pos[a:b], 32, 10000.0, 1e-6) for a, b, w in segs])
    ref = orc.attention(orc.round_bf16(qn), as_input(raw["k"], torch.bfloat16)[0], as_input(raw["v"], torch.bfloat16)[0])
    assert_bf16(host(outs[0]).reshape(S, H, 128), ref, "attention with the q chain")
