"""Whole Flux2 blocks and a small Flux2 transformer on the GPU through the C++
host modules (Linear -> MUL_MAT, attention -> FLASH_ATTN_EXT, the
elementwise chain -> the fused kernels), against the oracle's fp32
composition of the same reference forward passes (oracle/flux2.py).

Weights are drawn N(0, 0.02) and rounded to bf16-representable values, and
activations are bf16-representable, so the fp32 reference and the bf16 device
path start from identical numbers; the device's error is then its bf16
activation roundings and fp32 accumulation order, held to the bf16 bar
(rel L2 <= 1e-2, cos >= 0.9999).  RMSNorm weights are N(1, 0.02) in fp32."""
import json
import os
import subprocess
import tempfile

import numpy as np
import pytest

from conftest import bf16_metrics
from test_gpu_fused import flux_positions
from test_gpu_host_cli import CLI, read_dtb, write_dtb

pytestmark = pytest.mark.gpu


def make_params(orc, shapes, seed0, bf16_weights=True):
    """Linear weights N(0, 0.02), rounded to bf16-representable values unless
    bf16_weights is False; RMSNorm weights N(1, 0.02) in fp32."""
    P = {}
    for i, (name, shape) in enumerate(sorted(shapes.items())):
        if len(shape) == 2:
            w = orc.randn(orc.tensor_seed(seed0 + i), shape, std=0.02)
            P[name] = orc.round_bf16(w) if bf16_weights else w
        else:
            P[name] = orc.randn(orc.tensor_seed(seed0 + i), shape, mean=1.0, std=0.02)
    return P


def write_params(d, P):
    wd = os.path.join(d, "weights")
    os.makedirs(wd, exist_ok=True)
    for name, a in P.items():
        write_dtb(os.path.join(wd, name + ".dtb"), np.asarray(a, np.float32), 0)
    return wd


def run_cli(command, *args, timeout=300):
    r = subprocess.run([CLI, command, *map(str, args)], capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, f"dit_cli {command} failed: {r.stderr}"
    return json.loads(r.stdout.strip().splitlines()[-1])


def check(got, want, what):
    rel, cos = bf16_metrics(got, want)
    print(f"  {what}: rel_l2={rel:.3e} cos={cos:.7f}", flush=True)
    assert rel <= 1e-2 and cos >= 0.9999, f"{what}: rel_l2={rel:.3e} cos={cos:.6f}"


@pytest.fixture
def tmp():
    with tempfile.TemporaryDirectory() as d:
        yield d


def _single_block_case(orc, tmp, S_txt, grid, D, heads, theta, dtype, txt_zero=False, bf16_weights=True):
    import oracle.flux2 as of
    pos = flux_positions(S_txt, grid)
    if txt_zero:
        pos[:S_txt] = 0
    S = pos.shape[0]
    P = make_params(orc, of.single_block_param_shapes(D, heads), 3000, bf16_weights)
    x = orc.randn(orc.tensor_seed(2990), (S, D))
    if bf16_weights:
        x = orc.round_bf16(x)
    cond = orc.randn(orc.tensor_seed(2991), (1, D))
    w_mod = orc.randn(orc.tensor_seed(2992), (3 * D, D), std=0.02)
    mod = orc.linear(of.silu(cond), w_mod)  # single_stream_modulation (SiLU + Linear)
    wd = write_params(tmp, P)
    xp, mp, pp, op = (os.path.join(tmp, n) for n in ("x.dtb", "mod.dtb", "pos.dtb", "out.dtb"))
    write_dtb(xp, x.reshape(1, S, D), 0)
    write_dtb(mp, mod.reshape(1, 3 * D), 0)
    write_dtb(pp, pos, 26)
    stats = run_cli("Flux2SingleTransformerBlock", "--heads", heads, "--theta", theta, *sum(
        (["--axes_dim", 32] for _ in range(4)), []), "--weights", wd, "--hidden_states", xp,
        "--temb_mod", mp, "--position_ids", pp, "--dtype", dtype, "--out", op)
    want = of.single_block(x, mod, pos, P, heads, float(theta), 32)
    return read_dtb(op).reshape(S, D), want, stats


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_single_block_small(orc, tmp, dtype):
    print(f"single block S=16+64 D=256 {dtype}", flush=True)
    got, want, stats = _single_block_case(orc, tmp, 16, 8, 256, 2, 2000, dtype)
    check(got, want, f"single block {dtype}")
    print(f"  {stats}", flush=True)
    # adaLN, 2x QK-RMSNorm+RoPE, SwiGLU, GEMM-accumulate and gated residual fused
    assert stats["fused_nodes"] > 0


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_single_block_full_size(orc, tmp, dtype):
    """One Flux2-style single-stream block: hidden 3072, 24 x 128 heads, MLP
    9216, 1536 tokens (512 text with zero positions, then a 32 x 32 image
    grid), theta 2000; modulation from a N(0, 1) conditioning vector through
    SiLU + Linear.  bf16: bf16-representable weights and inputs, bf16
    activations, the bf16 bar.  f32 (the reference's precision): fp32 weights
    N(0, 0.02) and inputs N(0, 1) as drawn, fp32 activations, the fp32 GEMM
    and attention, held to rel L2 <= 1e-5."""
    print(f"single block S=512+1024 D=3072 {dtype}", flush=True)
    got, want, stats = _single_block_case(orc, tmp, 512, 32, 3072, 24, 2000, dtype, txt_zero=True,
                                          bf16_weights=dtype == "bf16")
    if dtype == "bf16":
        check(got, want, f"single block 1536x3072 {dtype}")
    else:
        rel, cos = bf16_metrics(got, want)
        print(f"  single block 1536x3072 fp32: rel_l2={rel:.3e} cos={cos:.9f}", flush=True)
        assert rel <= 1e-5, f"single block fp32: rel_l2={rel:.3e}"


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_double_block_small(orc, tmp, dtype):
    import oracle.flux2 as of
    print(f"double block 16+64 D=256 {dtype}", flush=True)
    D, heads, n_txt, grid = 256, 2, 16, 8
    pos = flux_positions(n_txt, grid)
    n_img = grid * grid
    P = make_params(orc, of.double_block_param_shapes(D, heads), 4000)
    h = orc.round_bf16(orc.randn(orc.tensor_seed(3990), (n_img, D)))
    e = orc.round_bf16(orc.randn(orc.tensor_seed(3991), (n_txt, D)))
    mi = orc.randn(orc.tensor_seed(3992), (6 * D,), std=0.5)
    mt = orc.randn(orc.tensor_seed(3993), (6 * D,), std=0.5)
    wd = write_params(tmp, P)
    f = {n: os.path.join(tmp, n + ".dtb") for n in ("h", "e", "mi", "mt", "pos", "oe", "oh")}
    write_dtb(f["h"], h.reshape(1, n_img, D), 0)
    write_dtb(f["e"], e.reshape(1, n_txt, D), 0)
    write_dtb(f["mi"], mi.reshape(1, -1), 0)
    write_dtb(f["mt"], mt.reshape(1, -1), 0)
    write_dtb(f["pos"], pos, 26)
    run_cli("Flux2TransformerBlock", "--heads", heads, "--theta", 2000,
            *sum((["--axes_dim", 32] for _ in range(4)), []), "--weights", wd, "--hidden_states", f["h"],
            "--encoder_hidden_states", f["e"], "--temb_mod_img", f["mi"], "--temb_mod_txt", f["mt"],
            "--position_ids", f["pos"], "--dtype", dtype, "--out-encoder", f["oe"], "--out-hidden", f["oh"])
    we, wh = of.double_block(h, e, mi, mt, pos, P, heads, 2000.0, 32)
    check(read_dtb(f["oh"]).reshape(n_img, D), wh, f"double block hidden {dtype}")
    check(read_dtb(f["oe"]).reshape(n_txt, D), we, f"double block encoder {dtype}")


SMALL_MODEL = dict(num_layers=1, num_single_layers=2, num_attention_heads=2, attention_head_dim=128,
                   in_channels=128, joint_attention_dim=128, timestep_guidance_channels=256, mlp_ratio=3.0,
                   rope_theta=2000, axes_dims_rope=[32, 32, 32, 32], eps=1e-6)


def _small_model_inputs(orc, tmp, n_txt=16, grid=8):
    n_img = grid * grid
    hid = orc.round_bf16(orc.randn(orc.tensor_seed(4990), (n_img, 128)))
    txt = orc.round_bf16(orc.randn(orc.tensor_seed(4991), (n_txt, 128)))
    pos = flux_positions(n_txt, grid)
    f = {n: os.path.join(tmp, n + ".dtb") for n in ("h", "t", "ts", "ii", "ti")}
    write_dtb(f["h"], hid.reshape(1, n_img, 128), 0)
    write_dtb(f["t"], txt.reshape(1, n_txt, 128), 0)
    write_dtb(f["ts"], np.array([0.5], np.float32), 0)
    write_dtb(f["ii"], pos[n_txt:], 26)
    write_dtb(f["ti"], pos[:n_txt], 26)
    return hid, txt, pos, f


def _run_small_model(f, wd, out, n_img, n_txt, *extra, layers=(1, 2)):
    return run_cli("Flux2Transformer2DModel", "--num_layers", layers[0], "--num_single_layers", layers[1],
                   "--num_attention_heads", 2, "--joint_attention_dim", 128, "--img_tokens", n_img,
                   "--txt_tokens", n_txt, "--weights", wd, "--hidden_states", f["h"],
                   "--encoder_hidden_states", f["t"], "--timestep", f["ts"], "--img_ids", f["ii"],
                   "--txt_ids", f["ti"], "--steps", 2, "--out", out, *extra)


def test_model_small(orc, tmp):
    """Flux2Transformer2DModel end to end at a small width: 1 double + 2
    single blocks, 2 x 128 heads, 64 image tokens (8 x 8) and 16 text tokens,
    timestep 0.5, no guidance embedding."""
    import oracle.flux2 as of
    cfg = SMALL_MODEL
    P = make_params(orc, of.model_param_shapes(cfg), 5000)
    hid, txt, pos, f = _small_model_inputs(orc, tmp)
    n_txt, n_img = txt.shape[0], hid.shape[0]
    out = os.path.join(tmp, "o.dtb")
    stats = _run_small_model(f, write_params(tmp, P), out, n_img, n_txt)
    print(f"  {stats}", flush=True)
    want = of.model(hid, txt, 0.5, pos[n_txt:], pos[:n_txt], P, cfg)
    check(read_dtb(out).reshape(n_img, 128), want, "model 1+2 blocks")


def test_model_small_node_order_alloc(orc, tmp):
    """--alloc node-order: node memory placed as ggml_gallocr places it (node
    order, in place where allowed), so the executor's address replay holds
    back fused launches that would read reused memory.  Held to the bf16 bar
    against the oracle like the fused placement."""
    import oracle.flux2 as of
    cfg = SMALL_MODEL
    P = make_params(orc, of.model_param_shapes(cfg), 5002)
    hid, txt, pos, f = _small_model_inputs(orc, tmp)
    n_txt, n_img = txt.shape[0], hid.shape[0]
    out = os.path.join(tmp, "o.dtb")
    stats = _run_small_model(f, write_params(tmp, P), out, n_img, n_txt, "--alloc", "node-order")
    print(f"  {stats}", flush=True)
    assert stats["alloc"] == "node-order"
    want = of.model(hid, txt, 0.5, pos[n_txt:], pos[:n_txt], P, cfg)
    check(read_dtb(out).reshape(n_img, 128), want, "model 1+2 blocks, node-order memory")


def test_model_small_hip_graph(orc, tmp):
    """--hip-graph true: the step is recorded once (dt_graph_capture) and
    replayed; after three replays, with the inputs uploaded again before each,
    the output equals the eager run's bit for bit."""
    import oracle.flux2 as of
    P = make_params(orc, of.model_param_shapes(SMALL_MODEL), 5001)
    hid, txt, pos, f = _small_model_inputs(orc, tmp)
    wd = write_params(tmp, P)
    eager, graph = os.path.join(tmp, "e.dtb"), os.path.join(tmp, "g.dtb")
    _run_small_model(f, wd, eager, hid.shape[0], txt.shape[0])
    st = _run_small_model(f, wd, graph, hid.shape[0], txt.shape[0], "--hip-graph", "true", "--warmup", 2)
    assert st["hip_graph"] is True
    a, b = read_dtb(eager), read_dtb(graph)
    assert a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_model_small_q8_0_weights(orc, tmp):
    """The same model with --weight-format q8_0: every Linear weight is
    quantised to Q8_0 on the device and repacked (DT_TYPE_Q8_0_SPLIT), and
    the MFMA GEMM dequantises inside its load path.  The output equals, bit
    for bit, the bf16 path run on the oracle's bf16 rounding of
    dequantize(quantize(W)), and is held to the bf16 bar against the
    oracle's fp32 model on those weights."""
    import oracle.flux2 as of
    cfg = SMALL_MODEL
    P = make_params(orc, of.model_param_shapes(cfg), 5000)
    Pq = {}
    for name, a in P.items():
        if a.ndim == 2:
            rows, cols = a.shape
            Pq[name] = orc.round_bf16(orc.dequantize(orc.quantize(a, 8), rows * cols, 8).reshape(rows, cols))
        else:
            Pq[name] = a
    hid, txt, pos, f = _small_model_inputs(orc, tmp)
    n_txt, n_img = txt.shape[0], hid.shape[0]
    qdir = os.path.join(tmp, "dequantized")
    os.makedirs(qdir)
    wq, wb = write_params(tmp, P), write_params(qdir, Pq)
    oq, ob = os.path.join(tmp, "oq.dtb"), os.path.join(tmp, "ob.dtb")
    sq = _run_small_model(f, wq, oq, n_img, n_txt, "--weight-format", "q8_0")
    print(f"  {sq}", flush=True)
    assert sq["weight_format"] == "q8_0"
    sb = _run_small_model(f, wb, ob, n_img, n_txt)
    assert sb["weight_format"] == "bf16"
    got_q, got_b = read_dtb(oq), read_dtb(ob)
    assert np.array_equal(got_q.view(np.uint32), got_b.view(np.uint32)), \
        f"Q8_0 path differs from bf16 on dequantised weights: max |d| {np.abs(got_q - got_b).max()}"
    want = of.model(hid, txt, 0.5, pos[n_txt:], pos[:n_txt], Pq, cfg)
    check(got_q.reshape(n_img, 128), want, "model 1+2 blocks, Q8_0 weights")


def _gguf_checkpoint(orc, tmp, P, type_of, fname):
    """P as a FLUX.2 GGUF checkpoint (fused tensors, per-tensor types) and the
    parameter values a reader decodes from it."""
    import gguf_writer as gw
    tensors, where = gw.fuse_flux2(P)
    items, decoded = [], {}
    for name, a in sorted(tensors.items()):
        raw, dec = gw.encode(orc, a, type_of(name, a))
        items.append((name, type_of(name, a), list(a.shape[::-1]), raw))
        decoded[name] = dec
    path = os.path.join(tmp, fname)
    gw.write_gguf(path, items, [("general.architecture", gw.STRING, "flux2")])
    return path, {p: gw.split_like(decoded[w[0]], w) for p, w in where.items()}


@pytest.mark.parametrize("weight_format", ["bf16", "q8_0"])
def test_model_small_from_gguf(orc, tmp, weight_format):
    """The small model from a GGUF checkpoint (dit_cli --gguf), the fused
    tensors split as the reference's loader splits them.  Linear weights are
    Q8_0, except (bf16 weights) x_embedder as BF16 and the second single
    block's to_out as Q4_K; norm weights F32, one F16 and one BF16.  The
    output equals, bit for bit, the same model run from --weights files
    holding the decoded values, and is held to the bf16 bar against the
    oracle on them."""
    import oracle.flux2 as of
    cfg = SMALL_MODEL
    P = make_params(orc, of.model_param_shapes(cfg), 5000)

    def type_of(name, a):
        if a.ndim == 1:
            if weight_format == "bf16" and name.endswith("blocks.0.attn.norm_q.weight"):
                return "F16"
            if weight_format == "bf16" and name.endswith("blocks.0.attn.norm_k.weight"):
                return "BF16"
            return "F32"
        if weight_format == "bf16" and name == "x_embedder.weight":
            return "BF16"
        if weight_format == "bf16" and name == "single_transformer_blocks.1.attn.to_out.weight":
            return "Q4_K"
        return "Q8_0"

    path, dec = _gguf_checkpoint(orc, tmp, P, type_of, "model.gguf")
    Pexp = {k: (orc.round_bf16(v) if v.ndim == 2 else v) for k, v in dec.items()}
    hid, txt, pos, f = _small_model_inputs(orc, tmp)
    n_txt, n_img = txt.shape[0], hid.shape[0]
    og, ow = os.path.join(tmp, "og.dtb"), os.path.join(tmp, "ow.dtb")
    sg = run_cli("Flux2Transformer2DModel", "--num_layers", 1, "--num_single_layers", 2,
                 "--num_attention_heads", 2, "--joint_attention_dim", 128, "--img_tokens", n_img,
                 "--txt_tokens", n_txt, "--gguf", path, "--hidden_states", f["h"],
                 "--encoder_hidden_states", f["t"], "--timestep", f["ts"], "--img_ids", f["ii"],
                 "--txt_ids", f["ti"], "--steps", 2, "--out", og, "--weight-format", weight_format)
    print(f"  {sg}", flush=True)
    assert sg["gguf_tensors_unused"] == 0 and sg["weight_format"] == weight_format
    wdir = os.path.join(tmp, "decoded")
    os.makedirs(wdir)
    # The files hold the decoded values themselves: the bf16 route rounds them
    # as dt_dequant does, the q8_0 route re-quantises d * q to the same blocks.
    sw = _run_small_model(f, write_params(wdir, dec), ow, n_img, n_txt, "--weight-format", weight_format)
    assert sw["kernels"] == sg["kernels"]
    got_g, got_w = read_dtb(og), read_dtb(ow)
    assert np.array_equal(got_g.view(np.uint32), got_w.view(np.uint32)), \
        f"GGUF path differs from the decoded weights: max |d| {np.abs(got_g - got_w).max()}"
    want = of.model(hid, txt, 0.5, pos[n_txt:], pos[:n_txt], Pexp, cfg)
    check(got_g.reshape(n_img, 128), want, f"model 1+2 blocks from GGUF ({weight_format})")
