"""The C++ host layer end to end, the way the reference's tests exercise its
modules: a Python test writes inputs, runs the command-line driver (here
diffusers-cpp_amd/bin/dit_cli, in the role of test/utils/*-cli), reads the
outputs and compares them with the oracle.  Cases follow the reference's
unit tests (test/src/nn/modules/normalization/{LayerNorm,GroupNorm,RMSNorm}.py,
test/src/nn/SiLU.py, test/src/diffusers/models/transformers/flux2/
{Flux2PosEmbed,Flux2SwiGLU}.py) plus Flux2-sized chains; graph statistics
printed by the driver confirm which node chains were fused."""
import json
import os
import subprocess
import tempfile

import numpy as np
import pytest

from conftest import PKG, assert_bf16, assert_fp32

pytestmark = pytest.mark.gpu

CLI = os.path.join(PKG, "bin", "dit_cli")
MAGIC = 0x31425444
SEED = 0x5EED2000


def write_dtb(path, a, type_):
    a = np.ascontiguousarray(a)
    with open(path, "wb") as f:
        f.write(np.array([MAGIC, type_, a.ndim, 0], dtype=np.int32).tobytes())
        f.write(np.array(a.shape, dtype=np.int64).tobytes())
        f.write(a.tobytes())


def read_dtb(path):
    with open(path, "rb") as f:
        hdr = np.frombuffer(f.read(16), dtype=np.int32)
        assert hdr[0] == MAGIC
        shape = tuple(np.frombuffer(f.read(8 * hdr[2]), dtype=np.int64))
        raw = f.read()
    if hdr[1] == 0:
        return np.frombuffer(raw, dtype=np.float32).reshape(shape)
    import oracle
    return oracle.from_bf16_bits(np.frombuffer(raw, dtype=np.uint16)).reshape(shape)


class Cli:
    def __init__(self, tmp, bf16=False):
        self.tmp = tmp
        self.bf16 = bf16
        self.n = 0

    def act(self, a):
        """An activation file; bf16 mode stores the RNE rounding and returns
        the values the device sees."""
        import oracle
        self.n += 1
        p = os.path.join(self.tmp, f"a{self.n}.dtb")
        if self.bf16:
            write_dtb(p, oracle.to_bf16_bits(a), 30)
            return p, oracle.round_bf16(a)
        write_dtb(p, np.asarray(a, np.float32), 0)
        return p, np.asarray(a, np.float32)

    def f32(self, a):
        self.n += 1
        p = os.path.join(self.tmp, f"p{self.n}.dtb")
        write_dtb(p, np.asarray(a, np.float32), 0)
        return p

    def i32(self, a):
        self.n += 1
        p = os.path.join(self.tmp, f"i{self.n}.dtb")
        write_dtb(p, np.asarray(a, np.int32), 26)
        return p

    def out(self, name="out"):
        return os.path.join(self.tmp, f"{name}.dtb")

    def run(self, command, *args):
        r = subprocess.run([CLI, command, *map(str, args)], capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, f"dit_cli {command} failed: {r.stderr}"
        return json.loads(r.stdout.strip().splitlines()[-1])


def check(got, want, bf16, what):
    if bf16:
        assert_bf16(got, want, what)
    else:
        assert_fp32(got, want, what=what)


@pytest.fixture(params=[False, True], ids=["f32", "bf16"])
def cli(request, dev):
    with tempfile.TemporaryDirectory() as d:
        yield Cli(d, bf16=request.param)


# ---- nn modules: the reference's own toy cases --------------------------------

def test_layernorm_affine_and_plain(orc, cli):
    x = orc.randn(SEED, (2, 2, 3))
    w = orc.randn(SEED + 1, (3,), mean=1.0, std=0.1)
    b = orc.randn(SEED + 2, (3,), std=0.1)
    xp, xv = cli.act(x)
    cli.run("LayerNorm", "--dim", 3, "--eps", "1e-5", "--x", xp, "--param-weight", cli.f32(w),
            "--param-bias", cli.f32(b), "--out", cli.out())
    want = orc.binary(0, orc.binary(2, orc.norm(xv, 1e-5), w), b)
    check(read_dtb(cli.out()), want, cli.bf16, "LayerNorm")
    cli.run("LayerNorm", "--dim", 3, "--eps", "1e-5", "--elementwise_affine", "false", "--x", xp,
            "--out", cli.out("o2"))
    check(read_dtb(cli.out("o2")), orc.norm(xv, 1e-5), cli.bf16, "LayerNorm no affine")


def test_rmsnorm_and_silu(orc, cli):
    x = orc.randn(SEED + 3, (4, 5, 40))
    w = orc.randn(SEED + 4, (40,), mean=1.0, std=0.02)
    xp, xv = cli.act(x)
    cli.run("RMSNorm", "--dim", 40, "--eps", "1e-6", "--x", xp, "--param-weight", cli.f32(w),
            "--out", cli.out())
    check(read_dtb(cli.out()), orc.binary(2, orc.rms_norm(xv, 1e-6), w), cli.bf16, "RMSNorm")
    st = cli.run("SiLU", "--x", xp, "--out", cli.out("s"))
    check(read_dtb(cli.out("s")), xv.astype(np.float64) / (1 + np.exp(-xv.astype(np.float64))), cli.bf16, "SiLU")
    assert st["kernels"] == 1 and st["fused_nodes"] == 1   # MUL(x, SIGMOID(x)) -> one kernel


@pytest.mark.parametrize("shape,G,affine,bias,silu", [
    ((2, 4, 3, 3), 2, True, True, False), ((1, 8, 4, 4), 4, True, True, False),
    ((2, 4, 2, 2), 2, False, False, False), ((2, 4, 2, 2), 2, True, False, False),
    ((1, 128, 32, 32), 32, True, True, True)])
def test_groupnorm(orc, cli, shape, G, affine, bias, silu):
    x = orc.randn(SEED + 5, shape)
    w = orc.randn(SEED + 6, (shape[1],), mean=1.0, std=0.02)
    b = orc.randn(SEED + 7, (shape[1],), std=0.02)
    xp, xv = cli.act(x)
    args = ["--num_groups", G, "--num_channels", shape[1], "--eps", "1e-6", "--input", xp,
            "--affine", str(affine).lower(), "--bias", str(bias).lower(), "--silu", str(silu).lower(),
            "--out", cli.out()]
    if affine:
        args += ["--param-weight", cli.f32(w)]
        if bias:
            args += ["--param-bias", cli.f32(b)]
    st = cli.run("GroupNorm", *args)
    want = orc.groupnorm_silu(xv, G, w if affine else None, b if affine and bias else None, 1e-6, silu=silu)
    check(read_dtb(cli.out()), want, cli.bf16, "GroupNorm")
    if affine and bias:
        assert st["kernels"] == 2, st        # stats + apply: the chain fused


def test_flux2_posembed_reference_cases(orc, cli):
    # Flux2PosEmbed.py test_zero / test_4d_axes: 4 axes x 2 dims, 4 heads
    for pos in (np.zeros((3, 4), np.int32), np.array([[0, 0, 0, 0], [1, 2, 3, 4], [5, 6, 7, 8]], np.int32)):
        x = orc.randn(SEED + 8, (1, 3, 4, 8))
        xp, xv = cli.act(x)
        cli.run("Flux2PosEmbed", "--theta", 10000, *sum((["--axes_dim", 2] for _ in range(4)), []),
                "--x", xp, "--position_ids", cli.i32(pos), "--out", cli.out())
        got = read_dtb(cli.out())
        want = np.concatenate([orc.rope_normal(xv[..., 2 * a:2 * a + 2], pos[:, a], 2, 10000.0)
                               for a in range(4)], -1)
        check(got, want, cli.bf16, "posembed")


@pytest.mark.parametrize("kind,message", [
    ("negative_dim", "needs more bytes than the file holds"),
    ("dims_overflow", "needs more bytes than the file holds"),
    ("short_payload", "needs more bytes than the file holds"),
    ("short_shape", "truncated tensor file"),
    ("element_type", "element type 8"),
])
def test_malformed_tensor_files_are_rejected(dev, kind, message):
    """A .dtb input whose header disagrees with its bytes (a negative or
    overflowing shape, a payload shorter than the shape, an element type the
    format does not carry) ends the command with a message, before any
    allocation sized by the header."""
    with tempfile.TemporaryDirectory() as d:
        good = os.path.join(d, "good.dtb")
        write_dtb(good, np.ones((2, 5, 48), np.float32), 0)
        bad = os.path.join(d, "bad.dtb")
        shape, type_, payload = [2, 5, 48], 0, np.ones(480, np.float32).tobytes()
        if kind == "negative_dim":
            shape = [2, -5, 48]
        elif kind == "dims_overflow":
            shape = [1 << 31, 1 << 31, 1 << 31]
        elif kind == "short_payload":
            payload = payload[:-4]
        elif kind == "element_type":
            type_ = 8
        with open(bad, "wb") as f:
            f.write(np.array([MAGIC, type_, len(shape), 0], dtype=np.int32).tobytes())
            if kind == "short_shape":   # the file ends inside the shape
                f.write(np.array(shape[:2], dtype=np.int64).tobytes())
            else:
                f.write(np.array(shape, dtype=np.int64).tobytes())
                f.write(payload)
        r = subprocess.run([CLI, "Flux2SwiGLU", "--gate", bad, "--up", good, "--out", os.path.join(d, "o.dtb")],
                           capture_output=True, text=True, timeout=120)
        assert r.returncode != 0, r.stdout
        assert message in r.stderr, r.stderr


def test_flux2_swiglu(orc, cli):
    g, u = orc.randn(SEED + 9, (2, 5, 48)), orc.randn(SEED + 10, (2, 5, 48))
    gp, gv = cli.act(g)
    up, uv = cli.act(u)
    st = cli.run("Flux2SwiGLU", "--gate", gp, "--up", up, "--out", cli.out())
    check(read_dtb(cli.out()), orc.swiglu(gv, uv), cli.bf16, "swiglu")
    assert st["kernels"] == 1


def test_adaln_modulation(orc, cli):
    x = orc.randn(SEED + 11, (1, 20, 3072))
    mod = orc.randn(SEED + 12, (1, 3 * 3072), std=0.1)
    xp, xv = cli.act(x)
    st = cli.run("AdaLNModulation", "--x", xp, "--mod", cli.f32(mod), "--out", cli.out())
    want = orc.adaln(xv[0], mod[0, :3072], mod[0, 3072:6144], 1e-6)
    check(read_dtb(cli.out())[0], want, cli.bf16, "adaln")
    # NORM/MUL/ADD and the FILL(1) + ADD(scale, 1) of the factor become one
    # kernel (the 1 is added to each scale as the kernel stages it)
    assert st["kernels"] == 1 and st["fused_nodes"] == 4, st


# ---- Flux2 chains at block shape ---------------------------------------------------

def seq_positions(n_txt, n_img, width):
    txt = [[0, 0, 0, l] for l in range(n_txt)]
    img = [[0, i // width, i % width, 0] for i in range(n_img)]
    return np.array(txt + img, dtype=np.int32)


def test_single_block_elementwise_chain(orc, cli):
    S, D, H, I = 96, 3072, 24, 9216
    pos = seq_positions(32, 64, 8)
    x, mod = orc.randn(SEED + 13, (1, S, D)), orc.randn(SEED + 14, (1, 3 * D), std=0.1)
    q, k = orc.randn(SEED + 15, (1, S, D)), orc.randn(SEED + 16, (1, S, D))
    g, u = orc.randn(SEED + 17, (1, S, I)), orc.randn(SEED + 18, (1, S, I))
    attn = orc.randn(SEED + 19, (1, S, D))
    wq = orc.randn(SEED + 20, (128,), mean=1.0, std=0.02)
    wk = orc.randn(SEED + 21, (128,), mean=1.0, std=0.02)
    xp, xv = cli.act(x)
    qp, qv = cli.act(q)
    kp, kv = cli.act(k)
    gp, gv = cli.act(g)
    upp, uv = cli.act(u)
    ap, av = cli.act(attn)
    st = cli.run("Flux2SingleBlockElementwise", "--heads", H, "--theta", 2000,
                 *sum((["--axes_dim", 32] for _ in range(4)), []),
                 "--x", xp, "--mod", cli.f32(mod), "--q", qp, "--k", kp, "--mlp_gate", gp, "--mlp_up", upp,
                 "--attn_out", ap, "--position_ids", cli.i32(pos), "--param-norm_q", cli.f32(wq),
                 "--param-norm_k", cli.f32(wk), "--out-norm", cli.out("n"), "--out-q", cli.out("q"),
                 "--out-k", cli.out("k"), "--out-mlp", cli.out("m"), "--out-residual", cli.out("r"))
    m = mod[0]
    check(read_dtb(cli.out("n"))[0], orc.adaln(xv[0], m[:D], m[D:2 * D], 1e-6), cli.bf16, "norm")
    check(read_dtb(cli.out("q"))[0], orc.qk_rmsnorm_rope(qv[0].reshape(S, H, 128), wq, pos, 32, 2000.0),
          cli.bf16, "q")
    check(read_dtb(cli.out("k"))[0], orc.qk_rmsnorm_rope(kv[0].reshape(S, H, 128), wk, pos, 32, 2000.0),
          cli.bf16, "k")
    check(read_dtb(cli.out("m"))[0], orc.swiglu(gv[0], uv[0]), cli.bf16, "swiglu")
    check(read_dtb(cli.out("r"))[0], orc.gated_residual(xv[0], av[0], m[2 * D:]), cli.bf16, "residual")
    # adaLN with its 1 + scale + 4 position CONTs (made once, shared by the
    # q and k calls of Flux2PosEmbed::forward) + (q, k and SwiGLU in one
    # launch) + residual
    assert st["kernels"] == 7, st
    assert st["arena_bytes"] < st["naive_bytes"] / 2, st


def test_double_stream_qk(orc, cli):
    St, Si, H = 16, 32, 3
    pos = seq_positions(St, Si, 8)
    qt, qi = orc.randn(SEED + 22, (1, St, 384)), orc.randn(SEED + 23, (1, Si, 384))
    wt = orc.randn(SEED + 24, (128,), mean=1.0, std=0.02)
    wi = orc.randn(SEED + 25, (128,), mean=1.0, std=0.02)
    tp, tv = cli.act(qt)
    ip, iv = cli.act(qi)
    st = cli.run("Flux2DoubleStreamQK", "--heads", H, "--theta", 10000, *sum((["--axes_dim", 32] for _ in range(4)), []),
                 "--txt_q", tp, "--img_q", ip, "--position_ids", cli.i32(pos),
                 "--param-norm_added_q", cli.f32(wt), "--param-norm_q", cli.f32(wi), "--out", cli.out())
    got = read_dtb(cli.out())[0]
    want = np.concatenate([orc.qk_rmsnorm_rope(tv[0].reshape(St, H, 128), wt, pos[:St], 32, 10000.0),
                           orc.qk_rmsnorm_rope(iv[0].reshape(Si, H, 128), wi, pos[St:], 32, 10000.0)])
    check(got, want, cli.bf16, "double-stream q")
    assert st["kernels"] == 4 + 2, st      # 4 position CONTs + one fused launch per segment


# ---- VAE decoder convolutions (test/src/nn/modules/conv/Conv2d.py,
# test/src/diffusers/models/resnet/Upsample2D.py) -------------------------------
# The conv multiplies bf16-rounded operands (fp32 accumulation), so the
# oracle runs on the rounded input and weights.

@pytest.mark.parametrize("x_shape,ci,co,k,pad,bias", [((1, 3, 8, 8), 3, 4, 3, 1, True),
                                                     ((1, 4, 5, 5), 4, 2, 1, 0, False),
                                                     ((2, 64, 20, 24), 64, 96, 3, 1, True)])
def test_conv2d(orc, cli, x_shape, ci, co, k, pad, bias):
    x = orc.randn(SEED + 40, x_shape)
    w = orc.randn(SEED + 41, (co, ci, k, k), std=0.2)
    b = orc.randn(SEED + 42, (co,), std=0.1)
    xp, xv = cli.act(x)
    args = ["--in_channels", ci, "--out_channels", co, "--kernel_size", k, "--stride", 1, "--padding", pad,
            "--bias", str(bias).lower(), "--x", xp, "--param-weight", cli.f32(w), "--out", cli.out()]
    if bias:
        args += ["--param-bias", cli.f32(b)]
    st = cli.run("Conv2d", *args)
    got = read_dtb(cli.out())
    want = orc.conv2d(orc.round_bf16(xv), orc.round_bf16(w), b if bias else None)
    check(got, want, cli.bf16, "Conv2d")
    assert st["fused_nodes"] == (1 if bias else 0), st      # the bias ADD folds into the conv
    assert st["kernels"] == (3 if k == 3 or cli.bf16 else 2), st  # pack, channel-last copy (3x3; 1x1 bf16), conv
    # the weight packed once at load (DT_TYPE_CONV2D_PACKED): no pack per call, same bits
    sp = cli.run("Conv2d", *args, "--packed-weights", "true")
    assert np.array_equal(read_dtb(cli.out()).view(np.uint32), got.view(np.uint32))
    assert sp["kernels"] == st["kernels"] - 1 and sp["fused_nodes"] == st["fused_nodes"], sp


def test_conv2d_stride_2_is_reported(orc, cli):
    """Conv2d.py test_stride2: strided convolutions (the VAE encoder's
    downsampling) are outside the decoder path and fail with a message."""
    xp, _ = cli.act(orc.randn(SEED + 43, (2, 3, 16, 16)))
    r = subprocess.run([CLI, "Conv2d", "--in_channels", "3", "--out_channels", "5", "--kernel_size", "3",
                        "--stride", "2", "--padding", "1", "--x", xp, "--param-weight",
                        cli.f32(np.zeros((5, 3, 3, 3))), "--param-bias", cli.f32(np.zeros(5)), "--out",
                        cli.out()], capture_output=True, text=True, timeout=60)
    assert r.returncode != 0 and "stride and dilation 1 only" in r.stderr, r.stderr


@pytest.mark.parametrize("use_conv,shape", [(False, (1, 4, 4, 4)), (True, (1, 4, 4, 4)), (True, (1, 128, 24, 20))])
def test_upsample2d(orc, cli, use_conv, shape):
    C = shape[1]
    x = orc.randn(SEED + 44, shape)
    w = orc.randn(SEED + 45, (C, C, 3, 3), std=0.05)
    b = orc.randn(SEED + 46, (C,), std=0.1)
    xp, xv = cli.act(x)
    args = ["--channels", C, "--use_conv", str(use_conv).lower(), "--hidden_states", xp, "--out", cli.out()]
    if use_conv:
        args += ["--param-conv.weight", cli.f32(w), "--param-conv.bias", cli.f32(b)]
    st = cli.run("Upsample2D", *args)
    got = read_dtb(cli.out())
    if not use_conv:
        assert np.array_equal(got, np.repeat(np.repeat(xv, 2, axis=2), 2, axis=3))
        assert st["kernels"] == 1, st
        return
    want = orc.conv2d(orc.round_bf16(xv), orc.round_bf16(w), b, up2=True)
    check(got, want, cli.bf16, "Upsample2D")
    assert st["fused_nodes"] == 2 and st["kernels"] == 3, st  # upscale + conv folded under the bias ADD
    sp = cli.run("Upsample2D", *args, "--packed-weights", "true")
    assert np.array_equal(read_dtb(cli.out()).view(np.uint32), got.view(np.uint32))
    assert sp["fused_nodes"] == 2 and sp["kernels"] == 2, sp


# ---- ResnetBlock2D (test/src/diffusers/models/resnet/ResnetBlock2D.py): the
# reference's three toy cases (groups 8 on a 1x8x2x2 input: 8 -> 8, the 8 -> 16
# channel projection, temb 16) and two decoder-sized blocks.  Interior
# activations are rounded to bf16 where they feed a convolution's MFMA (and,
# in bf16 mode, at every node), so both modes are held to the bf16 bar; f32
# mode is also compared, tighter, with the oracle rounding conv operands.

RESNET_CASES = [
    dict(cin=8, cout=8, temb=None, groups=8, N=1, H=2, W=2, osf=1.0),
    dict(cin=8, cout=16, temb=None, groups=8, N=1, H=2, W=2, osf=1.0),
    dict(cin=8, cout=8, temb=16, groups=8, N=1, H=2, W=2, osf=1.0),
    dict(cin=128, cout=128, temb=None, groups=32, N=1, H=24, W=40, osf=1.0),
    dict(cin=256, cout=128, temb=None, groups=32, N=1, H=16, W=20, osf=2.0),
]


@pytest.mark.parametrize("c", RESNET_CASES, ids=lambda c: f"{c['cin']}-{c['cout']}-t{c['temb']}-{c['H']}x{c['W']}")
def test_resnet_block2d(orc, cli, c):
    import oracle.vae as vae
    shapes = vae.resnet_block2d_param_shapes(c["cin"], c["cout"], c["temb"])
    wdir = os.path.join(cli.tmp, "w")
    os.makedirs(wdir, exist_ok=True)
    P = {}
    for i, (name, shape) in enumerate(sorted(shapes.items())):
        mean = 1.0 if name in ("norm1.weight", "norm2.weight") else 0.0
        std = 0.05 if name.endswith(".weight") and "norm" not in name else 0.1
        P[name] = orc.randn(SEED + 50 + i, shape, mean=mean, std=std)
        write_dtb(os.path.join(wdir, name + ".dtb"), P[name], 0)
    xp, xv = cli.act(orc.randn(SEED + 48, (c["N"], c["cin"], c["H"], c["W"])))
    args = ["--in_channels", c["cin"], "--out_channels", c["cout"], "--groups", c["groups"],
            "--output_scale_factor", c["osf"], "--dtype", "bf16" if cli.bf16 else "f32",
            "--hidden_states", xp, "--weights", wdir, "--out", cli.out()]
    tv = None
    if c["temb"]:
        tp, tv = cli.act(orc.randn(SEED + 49, (c["N"], c["temb"])))
        args += ["--temb_channels", c["temb"], "--temb", tp]
    st = cli.run("ResnetBlock2D", *args)
    got = read_dtb(cli.out())
    want = vae.resnet_block2d(xv, P, c["groups"], None, 1e-6, c["osf"], tv)
    assert_bf16(got, want, "ResnetBlock2D")
    if not cli.bf16:
        from conftest import bf16_metrics
        rel, _ = bf16_metrics(got, vae.resnet_block2d(xv, P, c["groups"], None, 1e-6, c["osf"], tv, conv_bf16=True))
        assert rel <= 2e-3, rel
    shortcut = c["cin"] != c["cout"]
    if not c["temb"]:
        # GroupNorm+SiLU 2 each; conv1 and conv2: pack, channel-last copy, conv (conv2 with
        # the bias, residual ADD and SCALE in its epilogue); the 1x1 shortcut: pack, conv
        # (and the channel-last copy on bf16)
        assert st["kernels"] == 10 + ((3 if cli.bf16 else 2) if shortcut else 0), st
    sp = cli.run("ResnetBlock2D", *args, "--packed-weights", "true")
    assert np.array_equal(read_dtb(cli.out()).view(np.uint32), got.view(np.uint32))
    assert sp["kernels"] == st["kernels"] - (3 if shortcut else 2), sp


@pytest.mark.parametrize("c", [dict(cin=8, cout=4, layers=2, groups=4, H=8, W=8, up=False),
                               dict(cin=8, cout=4, layers=2, groups=4, H=8, W=8, up=True),
                               dict(cin=128, cout=64, layers=3, groups=32, H=24, W=20, up=True)],
                         ids=lambda c: f"{c['cin']}-{c['cout']}-l{c['layers']}-up{int(c['up'])}")
def test_up_decoder_block2d(orc, cli, c):
    """UpDecoderBlock2D.py's two cases (8 -> 4, two layers, groups 4 on
    1x8x8x8, with and without the upsampler) and a decoder-sized block."""
    import oracle.vae as vae
    shapes = vae.up_decoder_block2d_param_shapes(c["cin"], c["cout"], c["layers"], c["up"])
    wdir = os.path.join(cli.tmp, "w")
    os.makedirs(wdir, exist_ok=True)
    P = {}
    for i, (name, shape) in enumerate(sorted(shapes.items())):
        mean = 1.0 if name.endswith(("norm1.weight", "norm2.weight")) else 0.0
        std = 0.05 if name.endswith(".weight") and "norm" not in name else 0.1
        P[name] = orc.randn(SEED + 80 + i, shape, mean=mean, std=std)
        write_dtb(os.path.join(wdir, name + ".dtb"), P[name], 0)
    xp, xv = cli.act(orc.randn(SEED + 79, (1, c["cin"], c["H"], c["W"])))
    args = ["--in_channels", c["cin"], "--out_channels", c["cout"], "--num_layers", c["layers"],
            "--resnet_groups", c["groups"], "--add_upsample", str(c["up"]).lower(),
            "--dtype", "bf16" if cli.bf16 else "f32", "--hidden_states", xp, "--weights", wdir, "--out", cli.out()]
    st = cli.run("UpDecoderBlock2D", *args)
    got = read_dtb(cli.out())
    want = vae.up_decoder_block2d(xv, P, c["layers"], c["groups"], 1e-6, 1.0, c["up"])
    assert got.shape == want.shape
    assert_bf16(got, want, "UpDecoderBlock2D")
    # per resnet: two GroupNorm folds (statistics, (mean, rstd)), conv1 and conv2 (pack,
    # channel-last copy, conv); the first block's 1x1 shortcut (pack, conv, and the copy on
    # bf16) and the upsampler (pack, copy, conv)
    shortcut = c["cin"] != c["cout"]
    assert st["kernels"] == 10 * c["layers"] + ((3 if cli.bf16 else 2) if shortcut else 0) + (3 if c["up"] else 0), st
    sp = cli.run("UpDecoderBlock2D", *args, "--packed-weights", "true")
    assert np.array_equal(read_dtb(cli.out()).view(np.uint32), got.view(np.uint32))
    n_convs = 2 * c["layers"] + (1 if shortcut else 0) + (1 if c["up"] else 0)
    assert sp["kernels"] == st["kernels"] - n_convs, sp


@pytest.mark.parametrize("block", ["ResnetBlock2D", "UpDecoderBlock2D"])
def test_decoder_blocks_under_node_order_allocation(dev, block):
    """With node memory placed as ggml's allocator would place it (node order,
    in place where the op allows: the residual ADD may land on its input),
    the GroupNorm-in-copy and residual-in-epilogue folds give the same bits
    as with the executor's own placement; the memory replay keeps apart
    whatever the placement would break."""
    common = ["--random-inputs", "3", "--random-weights", "4", "--height", "40", "--width", "48",
              "--dtype", "bf16", "--packed-weights", "true"]
    if block == "ResnetBlock2D":
        args = ["--in_channels", "64", "--out_channels", "32", "--groups", "32"] + common
    else:
        args = ["--in_channels", "64", "--out_channels", "32", "--num_layers", "2", "--resnet_groups", "32"] + common
    runs = []
    for alloc in ("fused", "node-order"):
        r = subprocess.run([CLI, block, *args, "--alloc", alloc], capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stderr
        runs.append(json.loads(r.stdout.strip().splitlines()[-1]))
    assert runs[0]["output"]["fnv64"] == runs[1]["output"]["fnv64"], runs
    assert runs[0]["output"]["nonfinite"] == 0


def test_cli_rejects_bad_input(dev):
    with tempfile.TemporaryDirectory() as d:
        r = subprocess.run([CLI, "NoSuchCommand"], capture_output=True, text=True, timeout=60)
        assert r.returncode != 0
        r = subprocess.run([CLI, "SiLU", "--x", os.path.join(d, "missing.dtb"), "--out", os.path.join(d, "o")],
                           capture_output=True, text=True, timeout=60)
        assert r.returncode != 0 and "cannot open" in r.stderr
