"""GPU parity of the fused entry points against the oracle, through the C ABI.

Inputs come from the oracle's seeded generator; bf16 inputs are the RNE
rounding of the draw and the oracle consumes exactly those values.  Bars:
fp32 element-wise |d| <= 1e-5 * max(|ref|, 1); bf16 relative L2 <= 1e-2 with
cosine >= 0.9999, plus a per-element bound of one bf16 ulp around the fp32
reference; dequantisation bit-exact."""
import numpy as np
import pytest
import torch

import dit_hip
from conftest import assert_bf16, assert_fp32

pytestmark = pytest.mark.gpu

SEED = 0x5EED0000


def dev_tensor(a: np.ndarray, dtype, device="cuda"):
    """Upload float32 data as `dtype` (bf16 via the oracle's RNE bits)."""
    import oracle
    if dtype == torch.bfloat16:
        bits = oracle.to_bf16_bits(a).view(np.int16)
        return torch.from_numpy(bits).to(device).view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)


def host(t):
    return t.float().cpu().numpy()


def as_input(a, dtype):
    """The values the device sees for `a` stored as `dtype`."""
    import oracle
    return oracle.round_bf16(a) if dtype == torch.bfloat16 else np.asarray(a, np.float32)


def check(got, ref, dtype, what, one_rounding=True):
    """bf16: the bf16 bar (rel L2 <= 1e-2, cos >= 0.9999) and, for a
    single fused kernel (one rounding of an fp32 result), at most one bf16
    ulp per element; fp32: |d| <= 1e-5 * max(|ref|, 1)."""
    if dtype == torch.bfloat16:
        assert_bf16(got, ref, what)
        if not one_rounding:
            return
        r = np.asarray(ref, np.float64)
        err = np.abs(np.asarray(got, np.float64) - r)
        bound = np.abs(r) * 2.0 ** -8 + 1e-5 * max(1.0, float(np.abs(r).max()))
        assert np.all(err <= bound), f"{what}: {int((err > bound).sum())} elements beyond 1 bf16 ulp"
    else:
        assert_fp32(got, ref, what=what)


DT = [torch.bfloat16, torch.float32]


# ------------------------------------------------------------------ adaLN -----
@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("rows,cols", [(4608, 3072), (37, 3072), (64, 1000), (5, 100), (3, 3)])
def test_adaln(orc, dev, dtype, rows, cols):
    print(f"adaln rows={rows} cols={cols} {dtype}", flush=True)
    x = orc.randn(SEED + 1, (rows, cols))
    sh = orc.randn(SEED + 2, (cols,), std=0.1)
    sc = orc.randn(SEED + 3, (cols,), std=0.1)
    xd = dev_tensor(x, dtype)
    y = dit_hip.adaln_mod(xd, dev_tensor(sh, torch.float32), dev_tensor(sc, torch.float32), 1e-6)
    torch.cuda.synchronize()
    check(host(y), orc.adaln(as_input(x, dtype), sh, sc, 1e-6), dtype, "adaln")


@pytest.mark.parametrize("dtype", DT)
def test_adaln_strided_and_inplace(orc, dev, dtype):
    rows, cols = 300, 3072
    big = orc.randn(SEED + 4, (rows, 4096))
    sh = orc.randn(SEED + 5, (cols,), std=0.1)
    sc = orc.randn(SEED + 6, (cols,), std=0.1)
    bd = dev_tensor(big, dtype)
    xv = bd[:, 512:512 + cols]                       # row stride 4096
    ref = orc.adaln(as_input(big[:, 512:512 + cols], dtype), sh, sc, 1e-6)
    dsh, dsc = dev_tensor(sh, torch.float32), dev_tensor(sc, torch.float32)
    y = dit_hip.adaln_mod(xv, dsh, dsc, 1e-6)
    torch.cuda.synchronize()
    check(host(y), ref, dtype, "adaln strided")
    dit_hip.adaln_mod(xv, dsh, dsc, 1e-6, out=xv)   # in place
    torch.cuda.synchronize()
    check(host(xv), ref, dtype, "adaln in-place")
    # columns outside the view are untouched
    assert np.array_equal(host(bd[:, :512]), as_input(big[:, :512], dtype))


# ------------------------------------------------------- QK RMSNorm + RoPE ----
def flux_positions(n_txt, grid):
    txt = np.array([[0, 0, 0, l] for l in range(n_txt)], dtype=np.int32)
    img = np.array([[0, y, x, 0] for y in range(grid) for x in range(grid)], dtype=np.int32)
    return np.concatenate([txt, img]).reshape(-1, 4)


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("use_table", [True, False])
def test_qk_rmsnorm_rope_full(orc, dev, dtype, use_table):
    # config: q, k [4608, 24, 128], text l < 512 then a 64x64 image grid, theta 1e4
    pos = flux_positions(512, 64)
    S, H, D = pos.shape[0], 24, 128
    print(f"qk S={S} {dtype} table={use_table}", flush=True)
    q = orc.randn(SEED + 10, (S, H, D))
    k = orc.randn(SEED + 11, (S, H, D))
    wq = orc.randn(SEED + 12, (D,), mean=1.0, std=0.02)
    wk = orc.randn(SEED + 13, (D,), mean=1.0, std=0.02)
    tab = dit_hip.rope_table(512, 32, 10000.0) if use_table else None
    qo, ko = dit_hip.qk_rmsnorm_rope(dev_tensor(q, dtype), dev_tensor(k, dtype),
                                     dev_tensor(wq, torch.float32), dev_tensor(wk, torch.float32),
                                     torch.from_numpy(pos).cuda(), 32, 10000.0, 1e-6, table=tab)
    torch.cuda.synchronize()
    check(host(qo), orc.qk_rmsnorm_rope(as_input(q, dtype), wq, pos, 32, 10000.0, 1e-6), dtype, "q")
    check(host(ko), orc.qk_rmsnorm_rope(as_input(k, dtype), wk, pos, 32, 10000.0, 1e-6), dtype, "k")


def test_qk_table_values_are_bit_exact(orc, dev):
    # With the host table the angles match the oracle exactly, so fp32
    # outputs differ only through the norm's reduction order (<= a few ulps).
    pos = flux_positions(16, 4)
    S = pos.shape[0]
    q = orc.randn(SEED + 14, (S, 2, 128))
    w = np.ones(128, np.float32)
    tab = dit_hip.rope_table(64, 32, 2000.0)
    qo, _ = dit_hip.qk_rmsnorm_rope(dev_tensor(q, torch.float32), None, dev_tensor(w, torch.float32),
                                    None, torch.from_numpy(pos).cuda(), 32, 2000.0, 1e-6, table=tab)
    ref = orc.qk_rmsnorm_rope(q, w, pos, 32, 2000.0, 1e-6)
    assert_fp32(host(qo), ref, tol=1e-6, what="qk table")


@pytest.mark.parametrize("dtype", DT)
def test_qk_strided_views_of_fused_projection(orc, dev, dtype):
    # q and k as column views of a fused [S, 3*3072] qkv output (token stride 9216)
    pos = flux_positions(40, 8)
    S = pos.shape[0]
    qkv = orc.randn(SEED + 15, (S, 3 * 3072))
    w = orc.randn(SEED + 16, (128,), mean=1.0, std=0.02)
    d = dev_tensor(qkv, dtype)
    q = d[:, :3072].unflatten(1, (24, 128))
    k = d[:, 3072:6144].unflatten(1, (24, 128))
    dw = dev_tensor(w, torch.float32)
    tab = dit_hip.rope_table(64, 32, 2000.0)
    pt = torch.from_numpy(pos).cuda()
    qo, ko = dit_hip.qk_rmsnorm_rope(q, k, dw, dw, pt, 32, 2000.0, 1e-6, table=tab, q_out=q, k_out=k)
    torch.cuda.synchronize()
    for part, off in (("q", 0), ("k", 3072)):
        x = as_input(qkv[:, off:off + 3072], dtype).reshape(S, 24, 128)
        check(host(d[:, off:off + 3072]).reshape(S, 24, 128),
              orc.qk_rmsnorm_rope(x, w, pos, 32, 2000.0, 1e-6), dtype, part)
    # v untouched
    assert np.array_equal(host(d[:, 6144:]), as_input(qkv[:, 6144:], dtype))


@pytest.mark.parametrize("dtype", DT)
def test_qk_generic_toy_shape_and_out_of_table_positions(orc, dev, dtype):
    # Flux2PosEmbed.py toy case: 4 axes x 2 dims, heads of 8.
    pos = np.array([[0, 0, 0, 0], [1, 2, 3, 4], [5, 6, 7, 8]], dtype=np.int32)
    x = orc.randn(SEED + 17, (3, 4, 8))
    w = orc.randn(SEED + 18, (8,), mean=1.0, std=0.02)
    xo, _ = dit_hip.qk_rmsnorm_rope(dev_tensor(x, dtype), None, dev_tensor(w, torch.float32), None,
                                    torch.from_numpy(pos).cuda(), 2, 10000.0, 1e-6,
                                    table=dit_hip.rope_table(4, 2, 10000.0))   # p >= 4 off-table
    torch.cuda.synchronize()
    check(host(xo), orc.qk_rmsnorm_rope(as_input(x, dtype), w, pos, 2, 10000.0, 1e-6), dtype, "toy")
    # head_dim 128 but positions beyond the table (and negative)
    pos2 = np.array([[0, -3, 700, 5], [1, 2, 3, 1000]], dtype=np.int32)
    x2 = orc.randn(SEED + 19, (2, 3, 128))
    w2 = orc.randn(SEED + 20, (128,), mean=1.0, std=0.02)
    xo2, _ = dit_hip.qk_rmsnorm_rope(dev_tensor(x2, dtype), None, dev_tensor(w2, torch.float32), None,
                                     torch.from_numpy(pos2).cuda(), 32, 10000.0, 1e-6,
                                     table=dit_hip.rope_table(16, 32, 10000.0))
    torch.cuda.synchronize()
    check(host(xo2), orc.qk_rmsnorm_rope(as_input(x2, dtype), w2, pos2, 32, 10000.0, 1e-6), dtype, "off")


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("n_txt,grid,heads,head_dim,inner", [
    (512, 64, 24, 128, 9216),   # single-stream block: q, k [4608, 24, 128], gate/up [4608, 9216]
    (7, 3, 2, 128, 40),         # ragged: 16 tokens, SwiGLU rows not a multiple of the block
    (3, 2, 4, 8, 6),            # head_dim 8: the generic QK path, two launches
])
def test_qk_rmsnorm_rope_swiglu(orc, dev, dtype, n_txt, grid, heads, head_dim, inner):
    """q and k QK-RMSNorm+RoPE plus the block's SwiGLU in one launch: every
    output bit-identical to the separate kernels, and within tolerance of
    the oracle."""
    pos = flux_positions(n_txt, grid)
    S = pos.shape[0]
    axis_dim = head_dim // 4
    print(f"qk+swiglu S={S} H={heads} D={head_dim} inner={inner} {dtype}", flush=True)
    q = orc.randn(SEED + 32, (S, heads, head_dim))
    k = orc.randn(SEED + 33, (S, heads, head_dim))
    wq = orc.randn(SEED + 34, (head_dim,), mean=1.0, std=0.02)
    wk = orc.randn(SEED + 35, (head_dim,), mean=1.0, std=0.02)
    gu = orc.randn(SEED + 36, (S, 2 * inner))
    dq, dk, dgu = dev_tensor(q, dtype), dev_tensor(k, dtype), dev_tensor(gu, dtype)
    dwq, dwk = dev_tensor(wq, torch.float32), dev_tensor(wk, torch.float32)
    pt = torch.from_numpy(pos).cuda()
    tab = dit_hip.rope_table(512, axis_dim, 10000.0)
    qo, ko, y = dit_hip.qk_rmsnorm_rope_swiglu(dq, dk, dwq, dwk, pt, axis_dim, 10000.0,
                                               dgu[:, :inner], dgu[:, inner:], 1e-6, table=tab)
    qs, ks = dit_hip.qk_rmsnorm_rope(dq, dk, dwq, dwk, pt, axis_dim, 10000.0, 1e-6, table=tab)
    ys = dit_hip.swiglu(dgu[:, :inner], dgu[:, inner:])
    torch.cuda.synchronize()
    assert torch.equal(qo, qs) and torch.equal(ko, ks), "fused q/k differ from the QK kernel"
    assert torch.equal(y, ys), "fused SwiGLU differs from the SwiGLU kernel"
    # k alone with the SwiGLU (the block's q taken by its attention)
    _, ko1, y1 = dit_hip.qk_rmsnorm_rope_swiglu(None, dk, None, dwk, pt, axis_dim, 10000.0,
                                                dgu[:, :inner], dgu[:, inner:], 1e-6, table=tab)
    torch.cuda.synchronize()
    assert torch.equal(ko1, ks) and torch.equal(y1, ys), "k-only fused launch differs"
    check(host(qo), orc.qk_rmsnorm_rope(as_input(q, dtype), wq, pos, axis_dim, 10000.0, 1e-6), dtype, "q")
    check(host(ko), orc.qk_rmsnorm_rope(as_input(k, dtype), wk, pos, axis_dim, 10000.0, 1e-6), dtype, "k")
    g, u = as_input(gu[:, :inner], dtype), as_input(gu[:, inner:], dtype)
    check(host(y), orc.swiglu(g, u), dtype, "swiglu")


@pytest.mark.parametrize("dtype", DT)
def test_qk_rmsnorm_rope_swiglu_with_an_empty_half(orc, dev, dtype):
    """The fused entry with zero SwiGLU rows runs the QK half alone, and with
    zero tokens the SwiGLU half alone: each equals its separate kernel bit
    for bit, and the empty half's outputs are left untouched."""
    pos = flux_positions(16, 8)
    S, H, inner = pos.shape[0], 24, 9216
    q = orc.randn(SEED + 37, (S, H, 128))
    k = orc.randn(SEED + 38, (S, H, 128))
    wq = orc.randn(SEED + 39, (128,), mean=1.0, std=0.02)
    gu = orc.randn(SEED + 40, (S, 2 * inner))
    dq, dk, dgu = dev_tensor(q, dtype), dev_tensor(k, dtype), dev_tensor(gu, dtype)
    dw = dev_tensor(wq, torch.float32)
    pt = torch.from_numpy(pos).cuda()
    tab = dit_hip.rope_table(512, 32, 10000.0)
    qs, ks = dit_hip.qk_rmsnorm_rope(dq, dk, dw, dw, pt, 32, 10000.0, 1e-6, table=tab)
    ys = dit_hip.swiglu(dgu[:, :inner], dgu[:, inner:])
    # zero SwiGLU rows: q and k only
    y0 = torch.full((0, inner), 3.0, dtype=dtype, device="cuda")
    qo, ko, _ = dit_hip.qk_rmsnorm_rope_swiglu(dq, dk, dw, dw, pt, 32, 10000.0, dgu[:0, :inner], dgu[:0, inner:],
                                               1e-6, table=tab, out=y0)
    # zero tokens: the SwiGLU only; the (empty) q/k outputs are not touched
    qe = torch.full((0, H, 128), 3.0, dtype=dtype, device="cuda")
    _, _, y = dit_hip.qk_rmsnorm_rope_swiglu(dq[:0], dk[:0], dw, dw, pt[:0], 32, 10000.0, dgu[:, :inner],
                                             dgu[:, inner:], 1e-6, table=tab, q_out=qe, k_out=qe.clone())
    torch.cuda.synchronize()
    assert torch.equal(qo, qs) and torch.equal(ko, ks)
    assert torch.equal(y, ys)
    check(host(qo), orc.qk_rmsnorm_rope(as_input(q, dtype), wq, pos, 32, 10000.0, 1e-6), dtype, "q alone")


# ------------------------------------------------------------------ SwiGLU ----
@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("rows,inner", [(4608, 9216), (33, 3072), (5, 7)])
def test_swiglu_from_fused_gate_up(orc, dev, dtype, rows, inner):
    print(f"swiglu rows={rows} inner={inner} {dtype}", flush=True)
    gu = orc.randn(SEED + 21, (rows, 2 * inner))
    d = dev_tensor(gu, dtype)
    y = dit_hip.swiglu(d[:, :inner], d[:, inner:])
    torch.cuda.synchronize()
    g, u = as_input(gu[:, :inner], dtype), as_input(gu[:, inner:], dtype)
    check(host(y), orc.swiglu(g, u), dtype, "swiglu")


# ----------------------------------------------------------- gated residual ---
@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("rows,cols", [(4608, 3072), (17, 3072), (4, 13)])
def test_gated_residual(orc, dev, dtype, rows, cols):
    h = orc.randn(SEED + 22, (rows, cols))
    o = orc.randn(SEED + 23, (rows, cols))
    g = orc.randn(SEED + 24, (cols,), std=0.1)
    hd = dev_tensor(h, dtype)
    ref = orc.gated_residual(as_input(h, dtype), as_input(o, dtype), g)
    y = dit_hip.gated_residual(hd, dev_tensor(o, dtype), dev_tensor(g, torch.float32))
    torch.cuda.synchronize()
    check(host(y), ref, dtype, "gated")
    dit_hip.gated_residual(hd, dev_tensor(o, dtype), dev_tensor(g, torch.float32), out=hd)  # in place
    torch.cuda.synchronize()
    check(host(hd), ref, dtype, "gated in-place")


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("rows,cols", [(4608, 3072), (77, 3072), (3000, 1024), (40, 1000), (9, 512), (6, 6144),
                                       (5, 8192), (7, 1001)])
def test_gated_residual_adaln(orc, dev, dtype, rows, cols):
    """Block i's residual r = h + gate * o feeding block i+1's adaLN, one
    pass.  Reference: the oracle's gated residual, rounded to the I/O type as
    the stored ADD node is, then the oracle's adaLN of that r.  Rows of 8192
    fp32 and 1001 columns take the two-launch path."""
    print(f"residual+adaln rows={rows} cols={cols} {dtype}", flush=True)
    h = orc.randn(SEED + 27, (rows, cols))
    o = orc.randn(SEED + 28, (rows, cols))
    g = orc.randn(SEED + 29, (cols,), std=0.1)
    sh = orc.randn(SEED + 30, (cols,), std=0.1)
    sc = orc.randn(SEED + 31, (cols,), std=0.1)
    f = lambda a: dev_tensor(a, torch.float32)
    r, y = dit_hip.gated_residual_adaln(dev_tensor(h, dtype), dev_tensor(o, dtype), f(g), f(sh), f(sc), 1e-6)
    torch.cuda.synchronize()
    r_ref = orc.gated_residual(as_input(h, dtype), as_input(o, dtype), g)
    check(host(r), r_ref, dtype, "residual")
    r_stored = as_input(r_ref, dtype)
    # the stored r must be bit-identical to the standalone gated residual kernel
    r_alone = dit_hip.gated_residual(dev_tensor(h, dtype), dev_tensor(o, dtype), f(g))
    torch.cuda.synchronize()
    assert torch.equal(r, r_alone), "fused residual differs from the standalone kernel"
    # and y bit-identical to the standalone adaLN of that r (same reduction
    # order), which also pins that every row is written exactly once
    y_alone = dit_hip.adaln_mod(r_alone, f(sh), f(sc), 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(y, y_alone), "fused adaLN differs from the standalone kernel"
    check(host(y), orc.adaln(host(r), sh, sc, 1e-6), dtype, "adaln of r")
    check(host(y), orc.adaln(r_stored, sh, sc, 1e-6), dtype, "adaln of oracle r", one_rounding=False)


@pytest.mark.parametrize("dtype", DT)
def test_euler_step(orc, dev, dtype):
    x = orc.randn(SEED + 25, (4096, 128))
    v = orc.randn(SEED + 26, (4096, 128))
    y = dit_hip.euler_step(dev_tensor(x, dtype), dev_tensor(v, dtype), -0.0625)
    torch.cuda.synchronize()
    check(host(y), orc.euler(as_input(x, dtype), as_input(v, dtype), -0.0625), dtype, "euler")


# ------------------------------------------------------------- GroupNorm ------
@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("shape", [(1, 512, 128, 128), (1, 512, 256, 256), (1, 256, 512, 512), (1, 128, 1024, 1024),
                                   (1, 512, 512, 512), (1, 256, 1024, 1024), (2, 64, 9, 7), (2, 4, 3, 3)])
@pytest.mark.parametrize("silu", [True, False])
def test_groupnorm_silu(orc, dev, dtype, shape, silu):
    """GroupNorm(32) + SiLU at every decoder map size: the four of the
    VAE-decoder workload and the decoder's [1,512,512,512] and
    [1,256,1024,1024] (Decoder.hpp:53-85), plus ragged small maps."""
    if shape[2] >= 256 and not silu:
        pytest.skip("large shapes covered with SiLU")
    print(f"groupnorm {shape} {dtype} silu={silu}", flush=True)
    G = 32 if shape[1] % 32 == 0 else 2
    x = orc.randn(SEED + 27, shape)
    w = orc.randn(SEED + 28, (shape[1],), mean=1.0, std=0.02)
    b = orc.randn(SEED + 29, (shape[1],), std=0.02)
    y = dit_hip.groupnorm_silu(dev_tensor(x, dtype), G, dev_tensor(w, torch.float32),
                               dev_tensor(b, torch.float32), 1e-6, silu=silu)
    torch.cuda.synchronize()
    check(host(y), orc.groupnorm_silu(as_input(x, dtype), G, w, b, 1e-6, silu=silu), dtype, "gn")


@pytest.mark.parametrize("dtype", DT)
def test_groupnorm_no_affine_inplace_and_offset_mean(orc, dev, dtype):
    x = orc.randn(SEED + 30, (1, 64, 32, 32), mean=50.0, std=0.5)   # large mean: cancellation
    ref = orc.groupnorm_silu(as_input(x, dtype), 32, None, None, 1e-6, silu=True)
    xd = dev_tensor(x, dtype)
    dit_hip.groupnorm_silu(xd, 32, None, None, 1e-6, silu=True, out=xd)
    torch.cuda.synchronize()
    check(host(xd), ref, dtype, "gn in-place")


# ----------------------------------------------------------- dequantisation ---
@pytest.mark.parametrize("qtype", [dit_hip.Q8_0, dit_hip.Q4_K])
@pytest.mark.parametrize("rows,cols", [(3072, 9216), (9216, 3072), (3072, 3072), (2048, 3072), (96, 9216),
                                       (9216, 256), (3001, 3072), (2001, 3072)])
def test_dequant_bit_exact(orc, dev, qtype, rows, cols):
    """The dense tensors run with a run length chosen by size: on 256 CUs
    the two full-size shapes take 8 blocks per run (the flat kernels), 3072^2
    and 3001 x 3072 take 4 and 2048 x 3072 and 2001 x 3072 take 2 (the
    two-half kernels; 3001 and 2001 rows end in a partial run), the two
    narrow shapes 1; every run length gives ggml's bits."""
    print(f"dequant q{qtype} {rows}x{cols}", flush=True)
    w = orc.randn(SEED + 31, (rows, cols), std=0.02)
    blocks = orc.quantize(w, qtype)
    ref = orc.dequantize(blocks, w.size, qtype).reshape(rows, cols)
    src = torch.from_numpy(blocks).cuda()
    y32 = dit_hip.dequant(src, qtype, rows, cols, torch.float32)
    ybf = dit_hip.dequant(src, qtype, rows, cols, torch.bfloat16)
    torch.cuda.synchronize()
    assert np.array_equal(y32.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(ybf.cpu().view(torch.int16).numpy().view(np.uint16), orc.to_bf16_bits(ref))


@pytest.mark.parametrize("qtype", [dit_hip.Q8_0, dit_hip.Q4_K])
def test_dequant_strided_output_rows(orc, dev, qtype):
    """Output rows wider than the tensor (one row per workgroup run, not the
    dense stream): same bits, and nothing written past each row."""
    rows, cols = 33, 3072
    blocks = orc.quantize(orc.randn(SEED + 39, (rows, cols), std=0.02), qtype)
    ref = orc.dequantize(blocks, rows * cols, qtype).reshape(rows, cols)
    y = torch.full((rows, cols + 64), 7.0, dtype=torch.float32, device="cuda")
    dit_hip.dequant(torch.from_numpy(blocks).cuda(), qtype, rows, cols, out=y[:, :cols])
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert np.array_equal(got[:, :cols].view(np.uint32), ref.view(np.uint32))
    assert (got[:, cols:] == 7.0).all()


def test_dequant_q8_0_unaligned_rows(orc, dev):
    """Rows of 3 blocks (102 bytes, not a multiple of 16) and a source at a
    2-byte offset take the per-lane gather path: same bits."""
    rows, cols = 37, 96
    blocks = orc.quantize(orc.randn(SEED + 38, (rows, cols), std=0.02), dit_hip.Q8_0)
    ref = orc.dequantize(blocks, rows * cols, dit_hip.Q8_0).reshape(rows, cols)
    for off in (0, 2):
        buf = torch.zeros(blocks.size + 16, dtype=torch.uint8, device="cuda")
        buf[off:off + blocks.size] = torch.from_numpy(blocks).cuda()
        y = dit_hip.dequant(buf[off:off + blocks.size], dit_hip.Q8_0, rows, cols, torch.float32)
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy().view(np.uint32), ref.view(np.uint32)), off


def test_dequant_q8_0_exhaustive(orc, dev):
    # every fp16 scale pattern x every int8 code: 65536 blocks of 32 -> 8 blocks per d
    d = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    blocks = np.zeros((65536, 8, 34), dtype=np.uint8)
    blocks[:, :, 0:2] = d.view(np.uint8).reshape(65536, 1, 2)
    blocks[:, :, 2:] = (np.arange(256, dtype=np.int32) - 128).astype(np.int8).view(np.uint8).reshape(8, 32)
    flat = blocks.reshape(-1)
    ref = orc.dequantize(flat, 65536 * 256, 8)
    y = dit_hip.dequant(torch.from_numpy(flat).cuda(), dit_hip.Q8_0, 65536, 256, torch.float32)
    got = y.cpu().numpy().reshape(-1)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_dequant_q4_K_random_bytes(orc, dev):
    # any byte pattern is a valid super-block: random headers, scales and codes
    rng = np.random.RandomState(7)
    nb = 4096
    blocks = rng.randint(0, 256, size=(nb, 144)).astype(np.uint8)
    # keep d/dmin finite so the comparison is about layout, not NaN payloads
    blocks[:, 1] &= 0x7B
    blocks[:, 3] &= 0x7B
    flat = blocks.reshape(-1)
    ref = orc.dequantize(flat, nb * 256, 12)
    y = dit_hip.dequant(torch.from_numpy(flat).cuda(), dit_hip.Q4_K, 16, nb * 256 // 16, torch.float32)
    assert np.array_equal(y.cpu().numpy().reshape(-1).view(np.uint32), ref.view(np.uint32))


def test_dequant_known_answer_blocks(dev):
    import json
    import os
    kat = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "quant_kat.json")))
    for key, qt, qk in (("q8_0", dit_hip.Q8_0, 32), ("q4_K", dit_hip.Q4_K, 256)):
        for case in kat[key]:
            blk = np.frombuffer(bytes.fromhex(case["block"]), dtype=np.uint8).copy()
            y = dit_hip.dequant(torch.from_numpy(blk).cuda(), qt, 1, qk, torch.float32)
            assert np.array_equal(y.cpu().numpy().reshape(-1).view(np.uint32),
                                  np.array(case["expected_f32_bits"], np.uint32)), key
