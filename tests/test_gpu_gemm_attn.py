"""GPU parity of the step-time kernels (Linear GEMM with bf16 or Q8_0
weights, attention) and the Q8_0 quantiser against the oracle, through the C
ABI.

Bars: the GEMM with fp32 output is held to |d| <= 1e-5 * max(|ref|, 1) (its
products of bf16 inputs are exact in fp32 and only the accumulation order
differs from the oracle's); bf16 outputs to the bf16 bar (rel L2 <= 1e-2,
cos >= 0.9999) plus one bf16 ulp for a single rounding.  Attention rounds its
softmax weights to bf16 before the PV product, so both of its output types are
held to the bf16 bar.  The quantiser is bit-exact."""
import numpy as np
import pytest
import torch

import dit_hip
from conftest import assert_bf16, assert_fp32, bf16_metrics
from test_gpu_fused import SEED, as_input, check, dev_tensor, host

pytestmark = pytest.mark.gpu


# ---------------------------------------------------------------- quantiser --
def _quant_rows(orc):
    x = orc.randn(SEED + 200, (61, 3072), std=0.02)
    x[0] = 0.0                                            # d = 0 -> id = 0
    x[1] = orc.randn(SEED + 201, (3072,), std=1e-6)       # subnormal fp16 d
    x[2] = orc.randn(SEED + 202, (3072,), std=300.0)
    # exact halves: amax 127 -> d = 1, so x * id = x and roundf rounds away from 0
    x[3] = np.tile(np.array([127.0, 0.5, 1.5, -2.5, -0.5, 2.5, 126.5, -126.5], np.float32), 384)
    return x


def test_quantize_q8_0_bit_exact(orc, dev):
    print("quantize_q8_0 61x3072", flush=True)
    x = _quant_rows(orc)
    got = dit_hip.quantize_q8_0(dev_tensor(x, torch.float32))
    torch.cuda.synchronize()
    want = orc.quantize(x, 8).reshape(x.shape[0], -1)
    g = got.cpu().numpy()
    assert g.shape == want.shape
    bad = np.argwhere(g != want)
    assert bad.size == 0, f"{len(bad)} bytes differ, first at {bad[0]}"


def test_quantize_q8_0_strided_rows(orc, dev):
    x = orc.randn(SEED + 203, (33, 1024), std=0.02)
    big = dev_tensor(np.concatenate([x, np.zeros((33, 64), np.float32)], axis=1), torch.float32)
    out = torch.zeros((33, 1024 // 32 * 34 + 6), dtype=torch.uint8, device="cuda")
    dit_hip.quantize_q8_0(big[:, :1024], out=out)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    assert np.array_equal(o[:, :1088], orc.quantize(x, 8).reshape(33, -1))
    assert not o[:, 1088:].any(), "wrote past the row"


# --------------------------------------------------------------------- GEMM --
GEMM_SHAPES = [(1, 64, 64), (130, 200, 320), (256, 256, 3072), (513, 1000, 128), (64, 33, 192)]


@pytest.mark.parametrize("config", [-1, 0, 1, 2, 5, 6, 8])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
def test_gemm(orc, dev, M, N, K, out_dtype, config):
    print(f"gemm M={M} N={N} K={K} {out_dtype} config={config}", flush=True)
    a = orc.randn(SEED + 210, (M, K))
    b = orc.randn(SEED + 211, (N, K), std=0.02)
    y = dit_hip.gemm(dev_tensor(a, torch.bfloat16), dev_tensor(b, torch.bfloat16), out_dtype=out_dtype,
                     config=config)
    torch.cuda.synchronize()
    ref = orc.linear(orc.round_bf16(a), orc.round_bf16(b))
    check(host(y), ref, out_dtype, f"gemm {M}x{N}x{K}")


@pytest.mark.parametrize("config", [0, 1, 2, 5, 6, 8])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_gemm_strided_bias_addend(orc, dev, out_dtype, config):
    M, N, K = 300, 384, 512
    big_a = orc.randn(SEED + 212, (M, K + 128))
    b = orc.randn(SEED + 213, (N, K), std=0.02)
    bias = orc.randn(SEED + 214, (N,), std=0.1)
    add = orc.randn(SEED + 215, (M, N + 8))
    ad = dev_tensor(big_a, torch.bfloat16)[:, 64:64 + K]           # lda = K + 128
    addd = dev_tensor(add, out_dtype)[:, :N]                        # ldd = N + 8
    out = torch.zeros((M, N + 16), dtype=out_dtype, device="cuda")
    dit_hip.gemm(ad, dev_tensor(b, torch.bfloat16), bias=dev_tensor(bias, torch.float32),
                 addend=addd, out=out[:, :N], config=config)
    torch.cuda.synchronize()
    lin = orc.linear(orc.round_bf16(big_a[:, 64:64 + K]), orc.round_bf16(b), bias)
    ref = lin + as_input(add[:, :N], out_dtype)
    got = host(out)
    check(got[:, :N], ref, out_dtype, "gemm strided+bias+addend")
    assert not got[:, N:].any(), "wrote past N"


def test_gemm_in_place_addend(orc, dev):
    """C aliasing the addend: y += x W^T, the accumulate form of the
    attention-plus-MLP output projection."""
    M, N, K = 200, 256, 256
    a, b = orc.randn(SEED + 216, (M, K)), orc.randn(SEED + 217, (N, K), std=0.02)
    c0 = orc.randn(SEED + 218, (M, N))
    c = dev_tensor(c0, torch.float32)
    dit_hip.gemm(dev_tensor(a, torch.bfloat16), dev_tensor(b, torch.bfloat16), addend=c, out=c)
    torch.cuda.synchronize()
    assert_fp32(host(c), orc.linear(orc.round_bf16(a), orc.round_bf16(b)) + c0, what="gemm in-place")


@pytest.mark.parametrize("config", [0, 1, 2, 5, 6, 8])
def test_gemm_large_sampled_rows(orc, dev, config):
    """4608 x 3072 x 3072 (a Flux2 block's attention projection); 88 rows
    spread over every row tile are checked against the oracle."""
    M, N, K = 4608, 3072, 3072
    a = orc.randn(SEED + 219, (M, K))
    b = orc.randn(SEED + 220, (N, K), std=0.02)
    y = dit_hip.gemm(dev_tensor(a, torch.bfloat16), dev_tensor(b, torch.bfloat16), out_dtype=torch.float32,
                     config=config)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([np.arange(0, M, 53), [M - 1]]))
    ref = orc.linear(orc.round_bf16(a[rows]), orc.round_bf16(b))
    assert_fp32(host(y)[rows], ref, what="gemm 4608x3072x3072")


@pytest.mark.parametrize("config", [-1, 0, 1, 2, 5, 6, 8])
def test_gemm_grouped(orc, dev, config):
    """Five GEMMs of different N and K (and an empty one) in one launch, each
    against the oracle: the q/k/v/gate/up pattern plus ragged edges."""
    shapes = [(300, 256, 256), (300, 384, 256), (300, 136, 320), (300, 520, 128), (0, 64, 64), (47, 72, 64)]
    items, refs = [], []
    for i, (M, N, K) in enumerate(shapes):
        a = orc.randn(SEED + 240 + i, (M, K))
        b = orc.randn(SEED + 250 + i, (N, K), std=0.02)
        items.append((dev_tensor(a, torch.bfloat16), dev_tensor(b, torch.bfloat16),
                      torch.zeros((M, N), dtype=torch.float32, device="cuda")))
        refs.append(orc.linear(orc.round_bf16(a), orc.round_bf16(b)) if M else np.zeros((0, N), np.float32))
    outs = dit_hip.gemm_grouped(items, config=config)
    torch.cuda.synchronize()
    for (M, N, K), o, r in zip(shapes, outs, refs):
        assert_fp32(host(o), r, what=f"grouped gemm {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K,lda_pad", [(64, 48, 16, 0), (300, 136, 40, 0), (33, 20, 3, 0), (129, 257, 200, 0),
                                           (70, 96, 64, 3), (1, 1, 1, 0)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_gemm_any_shape(orc, dev, M, N, K, lda_pad, out_dtype):
    """Shapes the tiled kernels do not take (ggml's mul_mat takes any K): K
    not a multiple of 64, a leading dimension that breaks 16-byte rows
    (lda = K + 3), single elements.  They run the masked kernel, against the
    oracle; an explicit tiled configuration refuses them."""
    print(f"gemm any M={M} N={N} K={K} lda=K+{lda_pad} {out_dtype}", flush=True)
    a = orc.randn(SEED + 230, (M, K + lda_pad))
    b = orc.randn(SEED + 231, (N, K), std=0.02)
    y = dit_hip.gemm(dev_tensor(a, torch.bfloat16)[:, :K], dev_tensor(b, torch.bfloat16), out_dtype=out_dtype)
    torch.cuda.synchronize()
    check(host(y), orc.linear(orc.round_bf16(a[:, :K]), orc.round_bf16(b)), out_dtype, f"gemm any {M}x{N}x{K}")
    y4 = dit_hip.gemm(dev_tensor(a, torch.bfloat16)[:, :K], dev_tensor(b, torch.bfloat16), out_dtype=out_dtype,
                      config=4)
    torch.cuda.synchronize()
    assert torch.equal(y4.view(torch.int16 if out_dtype == torch.bfloat16 else torch.int32),
                       y.view(torch.int16 if out_dtype == torch.bfloat16 else torch.int32))
    with pytest.raises(RuntimeError, match="K % 64 == 0"):
        dit_hip.gemm(dev_tensor(a, torch.bfloat16)[:, :K], dev_tensor(b, torch.bfloat16), config=0)


def test_gemm_any_shape_equals_tiled_on_tiled_shapes(orc, dev):
    """On a shape every kernel takes, the masked kernel accumulates k in the
    same order as the tiled ones (k-steps of 16, ascending): bit-identical C."""
    M, N, K = 200, 192, 256
    a = dev_tensor(orc.randn(SEED + 232, (M, K)), torch.bfloat16)
    b = dev_tensor(orc.randn(SEED + 233, (N, K), std=0.02), torch.bfloat16)
    outs = [dit_hip.gemm(a, b, out_dtype=torch.float32, config=c) for c in (0, 1, 2, 4, 5, 6, 8)]
    torch.cuda.synchronize()
    for c, o in zip((1, 2, 4, 5, 6, 8), outs[1:]):
        assert torch.equal(o.view(torch.int32), outs[0].view(torch.int32)), f"config {c}"
    z = torch.zeros((0, 64), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((8, 64), dtype=torch.bfloat16, device="cuda")
    assert dit_hip.gemm(z, w).shape == (0, 8)


# ------------------------------------------------------- Q8_0 weight GEMM --
def _q8_weight(orc, seed, N, K):
    """Q8_0 blocks of N(0, 0.02) weights (the device quantiser), their split
    layout and their bf16 dequantisation."""
    w = orc.randn(seed, (N, K), std=0.02)
    blocks = dit_hip.quantize_q8_0(dev_tensor(w, torch.float32))
    return blocks, dit_hip.q8_0_split(blocks, N, K), dit_hip.dequant(blocks, dit_hip.Q8_0, N, K)


def test_q8_0_split_layout(orc, dev):
    """codes = q + 128 as uint8 and scales = fp32(d) transposed, decoded from
    the block bytes on the host."""
    N, K = 37 * 4, 320
    blocks, q8, _ = _q8_weight(orc, SEED + 260, N, K)
    torch.cuda.synchronize()
    raw = blocks.cpu().numpy().reshape(N, K // 32, 34)
    d = raw[:, :, :2].copy().view(np.float16)[:, :, 0].astype(np.float32)
    qs = raw[:, :, 2:].view(np.int8).reshape(N, K)
    assert np.array_equal(q8.codes.cpu().numpy(), (qs.astype(np.int16) + 128).astype(np.uint8))
    assert np.array_equal(q8.scales.cpu().numpy(), d.T)


Q8_SHAPES = [(1, 64, 64), (130, 200, 320), (256, 256, 3072), (513, 1000, 128), (64, 33, 192), (300, 522, 256),
             (77, 130, 96), (40, 64, 32)]  # the last two: K % 64 == 32, the masked kernel


@pytest.mark.parametrize("config", [-1, 1, 3, 7, 9])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,N,K", Q8_SHAPES)
def test_gemm_q8_0_equals_dequant_then_gemm(orc, dev, M, N, K, out_dtype, config):
    """Dequantising in the GEMM's load path (config 3: 256 x 256 tiles in
    eight waves, converted after the LDS read; configs 7 and 9: the K = 64
    kernel's 256 x 256 tiles in four or eight waves and config 1: 128 x 128
    tiles, converted as they are staged; -1: picked by shape) gives the bf16 weights dt_dequant
    writes and the same fp32 accumulation order, so C is bit-identical to
    dt_dequant followed by the bf16 GEMM; and within the bar of the oracle on
    the dequantised weights."""
    if config != -1 and K % 64:
        pytest.skip("K % 64 == 32 runs the masked kernel only")
    print(f"gemm_q8_0 M={M} N={N} K={K} {out_dtype} config={config}", flush=True)
    a = orc.randn(SEED + 261, (M, K))
    _, q8, wd = _q8_weight(orc, SEED + 262, N, K)
    ad = dev_tensor(a, torch.bfloat16)
    if config == -1:
        y = dit_hip.gemm_q8_0(ad, q8, out_dtype=out_dtype)
    else:
        y = torch.empty((M, N), dtype=out_dtype, device="cuda")
        dit_hip.gemm_grouped([(ad, q8, y)], config=config)
    y_ref = dit_hip.gemm(ad, wd, out_dtype=out_dtype)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref), "Q8_0 GEMM differs from dequant + bf16 GEMM"
    check(host(y), orc.linear(orc.round_bf16(a), host(wd)), out_dtype, f"gemm_q8_0 {M}x{N}x{K}")


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_gemm_q8_0_bias_addend_strided(orc, dev, out_dtype):
    M, N, K = 300, 384, 512
    big_a = orc.randn(SEED + 263, (M, K + 128))
    _, q8, wd = _q8_weight(orc, SEED + 264, N, K)
    bias = dev_tensor(orc.randn(SEED + 265, (N,), std=0.1), torch.float32)
    add = dev_tensor(orc.randn(SEED + 266, (M, N + 8)), out_dtype)[:, :N]
    ad = dev_tensor(big_a, torch.bfloat16)[:, 64:64 + K]
    out = torch.zeros((M, N + 16), dtype=out_dtype, device="cuda")
    dit_hip.gemm_q8_0(ad, q8, bias=bias, addend=add, out=out[:, :N])
    ref = dit_hip.gemm(ad, wd, bias=bias, addend=add, out_dtype=out_dtype, config=2)
    torch.cuda.synchronize()
    assert torch.equal(out[:, :N], ref)
    assert not out[:, N:].any(), "wrote past N"


def test_gemm_q8_0_grouped_and_large(orc, dev):
    """The five projections of a single-stream block as one grouped Q8_0
    launch (4608 rows, N = 3072 x 3 + 9216 x 2, K = 3072), by the picked
    configuration and by the eight-wave kernel, bit-identical to the bf16
    grouped GEMM on the dequantised weights."""
    M, K = 4608, 3072
    a = dev_tensor(orc.randn(SEED + 267, (M, K)), torch.bfloat16)
    items_q, items_b = [], []
    for i, N in enumerate([3072, 3072, 3072, 9216, 9216]):
        _, q8, wd = _q8_weight(orc, SEED + 270 + i, N, K)
        items_q.append((a, q8, torch.empty((M, N), dtype=torch.bfloat16, device="cuda")))
        items_b.append((a, wd, torch.empty((M, N), dtype=torch.bfloat16, device="cuda")))
    outs_q = [o.clone() for o in dit_hip.gemm_grouped(items_q)]
    outs_q7 = [o.clone() for o in dit_hip.gemm_grouped(items_q, config=7)]
    outs_q3 = dit_hip.gemm_grouped(items_q, config=3)
    outs_b = dit_hip.gemm_grouped(items_b, config=2)
    torch.cuda.synchronize()
    for oq, oq7, oq3, ob in zip(outs_q, outs_q7, outs_q3, outs_b):
        assert torch.equal(oq, ob), "picked Q8_0 configuration"
        assert torch.equal(oq7, ob), "four-wave K = 64 Q8_0 kernel"
        assert torch.equal(oq3, ob), "eight-wave Q8_0 kernel"


def test_gemm_q8_0_rejects(orc, dev):
    a = torch.zeros((64, 64), dtype=torch.bfloat16, device="cuda")
    _, q8, wd = _q8_weight(orc, SEED + 280, 64, 64)
    with pytest.raises(RuntimeError, match="mixes Q8_0 and bf16"):
        dit_hip.gemm_grouped([(a, q8, torch.empty((64, 64), dtype=torch.bfloat16, device="cuda")),
                              (a, wd, torch.empty((64, 64), dtype=torch.bfloat16, device="cuda"))])
    with pytest.raises(RuntimeError, match="does not take Q8_0"):
        dit_hip.gemm_grouped([(a, q8, torch.empty((64, 64), dtype=torch.bfloat16, device="cuda"))], config=2)
    for config in (3, 7):
        with pytest.raises(RuntimeError, match="does not take bf16"):
            dit_hip.gemm_grouped([(a, wd, torch.empty((64, 64), dtype=torch.bfloat16, device="cuda"))],
                                 config=config)


# ---------------------------------------------------------------- attention --
def _attn_ref(orc, q, k, v, scale=None):
    """q [B, Sq, H, D] -> oracle attention per batch on the bf16-rounded values."""
    return np.stack([orc.attention(orc.round_bf16(q[i]), orc.round_bf16(k[i]), orc.round_bf16(v[i]), scale)
                     for i in range(q.shape[0])])


ATTN_SHAPES = [(1, 300, 300, 3), (2, 128, 64, 2), (1, 77, 500, 1), (1, 64, 1, 2), (1, 1, 129, 4)]


# ------------------------------------------------------------- fp32 path --
@pytest.mark.parametrize("M,N,K", [(1, 64, 64), (130, 200, 320), (256, 256, 3072), (77, 33, 40), (300, 136, 3),
                                   (129, 260, 12288)])
def test_gemm_f32(orc, dev, M, N, K):
    """F32 weights with F32 activations (the reference's own Linear precision)
    on the fp32 matrix cores, against the oracle's linear at the fp32 bar
    (|d| <= 1e-5 max(|ref|, 1)); with a bias and an addend; K of any size
    (3 and 40 take the masked loads)."""
    print(f"gemm_f32 M={M} N={N} K={K}", flush=True)
    a = orc.randn(SEED + 280, (M, K))
    b = orc.randn(SEED + 281, (N, K), std=0.02)
    bias = orc.randn(SEED + 282, (N,), std=0.1)
    add = orc.randn(SEED + 283, (M, N))
    y = dit_hip.gemm_f32(dev_tensor(a, torch.float32), dev_tensor(b, torch.float32),
                         bias=dev_tensor(bias, torch.float32), addend=dev_tensor(add, torch.float32))
    torch.cuda.synchronize()
    assert_fp32(host(y), orc.linear(a, b, bias) + add, what=f"gemm_f32 {M}x{N}x{K}")


def test_gemm_f32_strided_in_place(orc, dev):
    """lda = K + 4, C written into a wider buffer, and C aliasing the addend."""
    M, N, K = 200, 96, 256
    big_a = orc.randn(SEED + 284, (M, K + 4))
    b = orc.randn(SEED + 285, (N, K), std=0.02)
    c0 = orc.randn(SEED + 286, (M, N + 4))
    cd = dev_tensor(c0, torch.float32)
    dit_hip.gemm_f32(dev_tensor(big_a, torch.float32)[:, :K], dev_tensor(b, torch.float32), addend=cd[:, :N],
                     out=cd[:, :N])
    torch.cuda.synchronize()
    got = host(cd)
    assert_fp32(got[:, :N], orc.linear(big_a[:, :K], b) + c0[:, :N], what="gemm_f32 strided in place")
    assert np.array_equal(got[:, N:], c0[:, N:]), "wrote past N"


@pytest.mark.parametrize("B,Sq,Skv,H", ATTN_SHAPES + [(1, 1536, 1536, 24)])
def test_flash_attn_f32(orc, dev, B, Sq, Skv, H):
    """fp32 q, k, v (the reference's F32 attention): fp32 scores, softmax and
    products, against the oracle's attention at the fp32 bar; the last shape
    is the 1536-token single-stream block's."""
    print(f"attn_f32 B={B} Sq={Sq} Skv={Skv} H={H}", flush=True)
    q = orc.randn(SEED + 290, (B, Sq, H, 128))
    k = orc.randn(SEED + 291, (B, Skv, H, 128))
    v = orc.randn(SEED + 292, (B, Skv, H, 128))
    o = dit_hip.flash_attn_f32(dev_tensor(q, torch.float32), dev_tensor(k, torch.float32),
                               dev_tensor(v, torch.float32))
    torch.cuda.synchronize()
    ref = np.stack([orc.attention(q[i], k[i], v[i]) for i in range(B)])
    assert_fp32(host(o), ref, what=f"attn_f32 {B}x{Sq}x{Skv}x{H}")


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("B,Sq,Skv,H", ATTN_SHAPES)
def test_flash_attn(orc, dev, B, Sq, Skv, H, out_dtype):
    print(f"attn B={B} Sq={Sq} Skv={Skv} H={H} {out_dtype}", flush=True)
    q = orc.randn(SEED + 230, (B, Sq, H, 128))
    k = orc.randn(SEED + 231, (B, Skv, H, 128))
    v = orc.randn(SEED + 232, (B, Skv, H, 128))
    o = dit_hip.flash_attn(dev_tensor(q, torch.bfloat16), dev_tensor(k, torch.bfloat16),
                           dev_tensor(v, torch.bfloat16), out_dtype=out_dtype)
    torch.cuda.synchronize()
    ref = _attn_ref(orc, q, k, v)
    rel, cos = bf16_metrics(host(o), ref)
    print(f"  rel_l2={rel:.2e} cos={cos:.7f}", flush=True)
    assert_bf16(host(o), ref, f"attn {B}x{Sq}x{Skv}x{H}")


def test_flash_attn_fused_qkv_views(orc, dev):
    """q, k, v as column views of one [S, 3*H*128] projection output (token
    stride 3*H*128, head stride 128), output written into a wider buffer."""
    S, H = 257, 3
    qkv = orc.randn(SEED + 233, (S, 3 * H * 128))
    d = dev_tensor(qkv, torch.bfloat16).view(1, S, 3, H, 128)
    out = torch.zeros((1, S, H + 1, 128), dtype=torch.bfloat16, device="cuda")
    dit_hip.flash_attn(d[:, :, 0], d[:, :, 1], d[:, :, 2], out=out[:, :, :H])
    torch.cuda.synchronize()
    r = qkv.reshape(1, S, 3, H, 128)
    ref = _attn_ref(orc, r[:, :, 0], r[:, :, 1], r[:, :, 2])
    got = host(out)
    assert_bf16(got[:, :, :H], ref, "attn fused-qkv views")
    assert not got[:, :, H].any(), "wrote outside the heads"


def test_flash_attn_invariants(orc, dev):
    """Constant V rows give that constant back; scale 0 gives the mean of V."""
    S, H = 200, 2
    q = dev_tensor(orc.randn(SEED + 234, (1, S, H, 128)), torch.bfloat16)
    k = dev_tensor(orc.randn(SEED + 235, (1, S, H, 128)), torch.bfloat16)
    c = np.linspace(-2, 2, 128, dtype=np.float32)
    v_const = dev_tensor(np.broadcast_to(c, (1, S, H, 128)).copy(), torch.bfloat16)
    o = dit_hip.flash_attn(q, k, v_const, out_dtype=torch.float32)
    torch.cuda.synchronize()
    cb = as_input(c, torch.bfloat16)
    # sum_j p_j * c with sum_j p_j = 1 up to the bf16 rounding of each p_j
    assert np.allclose(host(o), np.broadcast_to(cb, (1, S, H, 128)), rtol=4e-3, atol=4e-3)
    v = orc.randn(SEED + 236, (1, S, H, 128))
    o0 = dit_hip.flash_attn(q, k, dev_tensor(v, torch.bfloat16), scale=0.0, out_dtype=torch.float32)
    torch.cuda.synchronize()
    mean = as_input(v, torch.bfloat16).mean(axis=1, keepdims=True)
    assert np.allclose(host(o0), np.broadcast_to(mean, o0.shape), rtol=1e-5, atol=1e-5)


def test_flash_attn_flux2_shape_sampled(orc, dev):
    """4608 tokens x 24 heads (a 1024^2 Flux2 step); two heads x 160 queries
    are checked against the oracle over all 4608 keys."""
    S, H = 4608, 24
    q = orc.randn(SEED + 237, (1, S, H, 128))
    k = orc.randn(SEED + 238, (1, S, H, 128))
    v = orc.randn(SEED + 239, (1, S, H, 128))
    o = host(dit_hip.flash_attn(dev_tensor(q, torch.bfloat16), dev_tensor(k, torch.bfloat16),
                                dev_tensor(v, torch.bfloat16)))
    rows = np.arange(0, S, 29)
    for h in (0, 17):
        ref = orc.attention(orc.round_bf16(q[0, rows, h:h + 1]), orc.round_bf16(k[0, :, h:h + 1]),
                            orc.round_bf16(v[0, :, h:h + 1]))
        assert_bf16(o[0, rows, h:h + 1], ref, f"attn 4608x24 head {h}")


# ---------------------------------------------- attention with the QK prologue --
# dt_flash_attn_qk_bf16 normalises and rotates q as it loads it.  Its q is
# built from the same operations in the same order as dt_qk_rmsnorm_rope's
# stored output, so the attention output is compared bit for bit with that
# kernel followed by dt_flash_attn_bf16 (and with the oracle at the bf16 bar).
from test_gpu_fused import flux_positions  # noqa: E402


def _qk_then_attn(q_segs, k, v, pos, table, axis_dim=32, base=10000.0, eps=1e-6, out_dtype=torch.bfloat16):
    B, _, H, D = q_segs[0][0].shape
    Sq = sum(q.shape[1] for q, _ in q_segs)
    qn = torch.empty((B, Sq, H, D), dtype=torch.bfloat16, device="cuda")
    t0 = 0
    for q, w in q_segs:
        n = q.shape[1]
        for b in range(B):
            dit_hip.qk_rmsnorm_rope(q[b], None, w, None, pos[t0:t0 + n], axis_dim, base, eps, table=table,
                                    q_out=qn[b, t0:t0 + n])
        t0 += n
    return dit_hip.flash_attn(qn, k, v, out_dtype=out_dtype), qn


PRO_CASES = [  # (B, txt, img, Skv, H, table n_pos or None)
    (1, 0, 300, 300, 3, 512), (2, 77, 223, 290, 2, 40), (1, 16, 48, 64, 1, None), (1, 5, 1, 129, 4, 512)]


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("B,n_txt,n_img,Skv,H,n_pos", PRO_CASES)
def test_flash_attn_qk_prologue_bit_exact(orc, dev, B, n_txt, n_img, Skv, H, n_pos, out_dtype):
    """One segment or txt | img with their own norm weights; q as column
    views of a wider projection; a table that covers every position, one
    that covers only some (the rest computed on the device), or none."""
    print(f"attn+qk B={B} txt={n_txt} img={n_img} Skv={Skv} H={H} n_pos={n_pos} {out_dtype}", flush=True)
    Sq = n_txt + n_img
    grid = max(1, int(np.ceil(np.sqrt(max(n_img, 1)))))
    img = [[0, i // grid, i % grid, 0] for i in range(n_img)]
    pos_np = np.array([[0, 0, 0, l] for l in range(n_txt)] + img, dtype=np.int32).reshape(Sq, 4)
    pos = torch.from_numpy(np.ascontiguousarray(pos_np)).cuda()
    table = dit_hip.rope_table(n_pos, 32, 10000.0) if n_pos else None
    proj = dev_tensor(orc.randn(SEED + 240, (B, Sq, 2 * H * 128)), torch.bfloat16).view(B, Sq, 2, H, 128)
    w_txt = dev_tensor(orc.randn(SEED + 241, (128,), mean=1.0, std=0.1), torch.float32)
    w_img = dev_tensor(orc.randn(SEED + 242, (128,), mean=1.0, std=0.1), torch.float32)
    segs = ([(proj[:, :n_txt, 1], w_txt)] if n_txt else []) + [(proj[:, n_txt:, 1], w_img)]
    k = dev_tensor(orc.randn(SEED + 243, (B, Skv, H, 128)), torch.bfloat16)
    v = dev_tensor(orc.randn(SEED + 244, (B, Skv, H, 128)), torch.bfloat16)
    got = dit_hip.flash_attn_qk(segs, k, v, pos, 32, 10000.0, table=table, out_dtype=out_dtype)
    want, qn = _qk_then_attn(segs, k, v, pos, table, out_dtype=out_dtype)
    torch.cuda.synchronize()
    assert torch.equal(got, want), f"max |d| {(got.float() - want.float()).abs().max().item():g}"
    if B == 1 and n_txt and n_img:  # and against the oracle's QK + attention
        x = host(proj)[0, :, 1]
        qo = np.concatenate([orc.qk_rmsnorm_rope(x[:n_txt], host(w_txt), pos_np[:n_txt], 32, 10000.0, 1e-6),
                             orc.qk_rmsnorm_rope(x[n_txt:], host(w_img), pos_np[n_txt:], 32, 10000.0, 1e-6)])
        ref = orc.attention(orc.round_bf16(qo), orc.round_bf16(host(k)[0]), orc.round_bf16(host(v)[0]))
        assert_bf16(host(got)[0], ref, "attn+qk vs oracle")


def test_flash_attn_qk_prologue_flux2_shape(orc, dev):
    """A single-stream block's attention at 1024^2: q [4608, 24, 128] taken
    from the fused projection before its norm, 512 txt + 64x64 img positions,
    theta 1e4, the host-built table: bit-identical to the two-kernel path."""
    S, H = 4608, 24
    pos_np = flux_positions(512, 64)
    pos = torch.from_numpy(pos_np).cuda()
    table = dit_hip.rope_table(512, 32, 10000.0)
    q = dev_tensor(orc.randn(SEED + 245, (1, S, H, 128)), torch.bfloat16)
    w = dev_tensor(orc.randn(SEED + 246, (128,), mean=1.0, std=0.02), torch.float32)
    k = dev_tensor(orc.randn(SEED + 247, (1, S, H, 128)), torch.bfloat16)
    v = dev_tensor(orc.randn(SEED + 248, (1, S, H, 128)), torch.bfloat16)
    got = dit_hip.flash_attn_qk([(q, w)], k, v, pos, 32, 10000.0, table=table)
    want, _ = _qk_then_attn([(q, w)], k, v, pos, table)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_flash_attn_qk_prologue_rejects(dev):
    z = torch.zeros((1, 8, 1, 128), dtype=torch.bfloat16, device="cuda")
    w = torch.ones(128, dtype=torch.float32, device="cuda")
    pos = torch.zeros((8, 4), dtype=torch.int32, device="cuda")
    with pytest.raises(dit_hip.DtError, match="axis_dim"):
        dit_hip.flash_attn_qk([(z, w)], z, z, pos, 24, 10000.0)      # 4 x 24 != 128
    with pytest.raises(dit_hip.DtError, match="axis_dim"):
        dit_hip.flash_attn_qk([(z, w)], z, z, pos[:, :2], 36, 10000.0)  # axis_dim % 8 != 0
