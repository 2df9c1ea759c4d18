"""GPU parity of the VAE decoder convolution (dt_conv2d) against the oracle's
conv_2d_direct + bias (oracle.conv2d), through the C ABI.

The conv rounds its operands to bf16 (as the Linear GEMM does), so the
reference is the oracle on the bf16-rounded input and weights: fp32 outputs
are held to |d| <= 1e-5 * max(|ref|, 1) (only the fp32 accumulation order
differs), bf16 outputs to the bf16 bar (rel L2 <= 1e-2, cos >= 0.9999) plus
one bf16 ulp for the single output rounding."""
import numpy as np
import pytest
import torch

import dit_hip
from test_gpu_fused import SEED, as_input, check, dev_tensor, host

pytestmark = pytest.mark.gpu

# (N, Ci, H, W), Co, K, upscale2: one tile; several output-channel tiles with
# a partial one and two input-channel chunks; 1x1; the upscale with a partial
# tile along the width; narrow images (16-wide tiles); a VAE mid-block shape.
SHAPES = [((1, 5, 7, 9), 4, 3, False), ((2, 40, 13, 70), 130, 3, False), ((1, 64, 16, 16), 64, 1, False),
          ((1, 32, 10, 33), 48, 3, True), ((1, 24, 5, 3), 16, 3, True), ((1, 512, 16, 32), 512, 3, False),
          ((1, 96, 9, 130), 32, 1, True), ((1, 40, 5, 300), 64, 3, False), ((1, 20, 40, 20), 24, 1, False)]


@pytest.mark.parametrize("ws", [True, None], ids=["dma", "staged"])
@pytest.mark.parametrize("io", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape,co,k,up2", SHAPES)
def test_conv2d(orc, dev, shape, co, k, up2, io, ws):
    """Both paths: with a workspace (channel-last copy, DMA-fed) and without."""
    print(f"conv2d x={shape} co={co} k={k} up2={up2} {io} ws={ws}", flush=True)
    x = orc.randn(SEED + 300, shape)
    w = orc.randn(SEED + 301, (co, shape[1], k, k), std=0.05)
    b = orc.randn(SEED + 302, (co,), std=0.1)
    wp = dit_hip.conv2d_pack(dev_tensor(w, torch.float32))
    y = dit_hip.conv2d(dev_tensor(x, io), wp, bias=dev_tensor(b, torch.float32), upscale2=up2, workspace=ws)
    torch.cuda.synchronize()
    ref = orc.conv2d(orc.round_bf16(as_input(x, io)), orc.round_bf16(w), b, up2=up2)
    assert tuple(y.shape) == ref.shape
    check(host(y), ref, io, f"conv2d {shape} -> {co} k{k}{' up2' if up2 else ''}")


def test_conv2d_bf16_weights_and_no_bias(orc, dev):
    """bf16 weights pack to the same operands as their fp32 values; no bias."""
    x = orc.randn(SEED + 303, (1, 48, 12, 20))
    w = orc.round_bf16(orc.randn(SEED + 304, (40, 48, 3, 3), std=0.05))
    y32 = dit_hip.conv2d(dev_tensor(x, torch.float32), dit_hip.conv2d_pack(dev_tensor(w, torch.float32)))
    y16 = dit_hip.conv2d(dev_tensor(x, torch.float32), dit_hip.conv2d_pack(dev_tensor(w, torch.bfloat16)))
    torch.cuda.synchronize()
    assert torch.equal(y32, y16)
    check(host(y32), orc.conv2d(orc.round_bf16(x), w), torch.float32, "conv2d no bias")


def test_conv2d_vae_shape_sampled(orc, dev):
    """[1, 128, 128, 128] -> 128 channels, 3x3 (the last up-block's resnet
    convs at 1/8 of the 1024^2 area): 16 output channels spread over both
    halves of the tile checked against the oracle."""
    x = orc.randn(SEED + 305, (1, 128, 128, 128))
    w = orc.randn(SEED + 306, (128, 128, 3, 3), std=0.03)
    b = orc.randn(SEED + 307, (128,), std=0.1)
    y = dit_hip.conv2d(dev_tensor(x, torch.bfloat16), dit_hip.conv2d_pack(dev_tensor(w, torch.float32)),
                       bias=dev_tensor(b, torch.float32))
    torch.cuda.synchronize()
    sel = np.arange(0, 128, 8)
    ref = orc.conv2d(orc.round_bf16(x), orc.round_bf16(w[sel]), b[sel])
    check(host(y)[:, sel], ref, torch.bfloat16, "conv2d 128x128x128 sampled")


def test_conv2d_rejects(dev):
    x = torch.zeros((1, 4, 8, 8), dtype=torch.float32, device="cuda")
    with pytest.raises(AssertionError):
        dit_hip.conv2d_pack(torch.zeros((4, 4, 5, 5), dtype=torch.float32, device="cuda"))
    wp = dit_hip.conv2d_pack(torch.zeros((4, 4, 3, 3), dtype=torch.float32, device="cuda"))
    wp.k = 5
    with pytest.raises(RuntimeError, match="kernel size 5 unsupported"):
        dit_hip.conv2d(x, wp)


# ---------------------------------------------- conv + GroupNorm statistics --
# (N, Ci, H, W), Co, K, upscale2, groups: the decoder's group sizes (16, 8, 4
# channels per group at 512, 256, 128 channels), a partial output-channel tile,
# partial pixel tiles, the upscale, 1x1, and one group per channel.
GN_CASES = [((1, 64, 12, 40), 512, 3, False, 32), ((2, 32, 9, 70), 256, 3, False, 32),
            ((1, 48, 16, 16), 128, 3, True, 32), ((1, 40, 7, 150), 192, 1, False, 48),
            ((1, 16, 5, 6), 64, 3, False, 64), ((1, 128, 64, 64), 128, 3, False, 32)]


@pytest.mark.parametrize("ws", [True, None], ids=["dma", "staged"])
@pytest.mark.parametrize("io", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape,co,k,up2,groups", GN_CASES)
def test_conv2d_gn_statistics_and_apply(orc, dev, shape, co, k, up2, groups, io, ws):
    """dt_conv2d_gn stores the same output as dt_conv2d and the (mean,
    variance) of each group of that stored output; dt_groupnorm_silu_from_stats
    then matches the oracle's GroupNorm+SiLU of the stored output (the fp32 /
    bf16 bar of one fused kernel) and the two-pass dt_groupnorm_silu on it."""
    print(f"conv2d_gn x={shape} co={co} k={k} up2={up2} groups={groups} {io} ws={ws}", flush=True)
    x = orc.randn(SEED + 310, shape)
    w = orc.randn(SEED + 311, (co, shape[1], k, k), std=0.05)
    b = orc.randn(SEED + 312, (co,), std=0.5)
    gw = orc.randn(SEED + 313, (co,), mean=1.0, std=0.1)
    gb = orc.randn(SEED + 314, (co,), std=0.1)
    wp = dit_hip.conv2d_pack(dev_tensor(w, torch.float32))
    xd, bd = dev_tensor(x, io), dev_tensor(b, torch.float32)
    y, stats = dit_hip.conv2d_gn(xd, wp, groups, bias=bd, upscale2=up2, workspace=ws)
    y_plain = dit_hip.conv2d(xd, wp, bias=bd, upscale2=up2, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(y, y_plain), "the statistics epilogue changed the stored output"
    yh = host(y).astype(np.float64)
    N = shape[0]
    mv = stats[: N * groups * 16].cpu().numpy().view(np.float64).reshape(N, groups, 2)
    grp = yh.reshape(N, groups, -1)
    assert np.allclose(mv[..., 0], grp.mean(axis=2), rtol=1e-6, atol=1e-6), "group means"
    assert np.allclose(mv[..., 1], grp.var(axis=2), rtol=1e-5, atol=1e-7), "group variances"
    gwd, gbd = dev_tensor(gw, torch.float32), dev_tensor(gb, torch.float32)
    out = dit_hip.groupnorm_silu_from_stats(y, stats, groups, gwd, gbd, eps=1e-6)
    torch.cuda.synchronize()
    ref = orc.groupnorm_silu(host(y), groups, gw, gb, eps=1e-6)
    check(host(out), ref, io, "GroupNorm+SiLU from conv statistics")
    ws = torch.empty(dit_hip.load().dt_groupnorm_workspace_bytes(N, co, yh[0, 0].size, groups), dtype=torch.uint8,
                     device="cuda")
    two_pass = dit_hip.groupnorm_silu(y, groups, gwd, gbd, eps=1e-6, workspace=ws)
    torch.cuda.synchronize()
    check(host(out), host(two_pass), io, "against the two-pass GroupNorm", one_rounding=False)


def test_conv2d_gn_rejects_groups_not_dividing_the_tile(dev):
    x = torch.zeros((1, 8, 8, 8), dtype=torch.float32, device="cuda")
    wp = dit_hip.conv2d_pack(torch.zeros((96, 8, 3, 3), dtype=torch.float32, device="cuda"))
    with pytest.raises(AssertionError):
        dit_hip.conv2d_gn(x, wp, 5)  # 96 % 5 != 0: no stats layout
    with pytest.raises(RuntimeError, match="must divide 128"):
        dit_hip.conv2d_gn(x, wp, 2)  # 48 channels per group


# ------------------------------------------------ through dt_graph_compute --
@pytest.fixture
def be(dev):
    from graphkit import Backend
    b = Backend()
    yield b.h
    torch.cuda.synchronize()
    b.close()


def _graph_conv(orc, io, shape, co, k, up, bias=True, seed=SEED + 320):
    from graphkit import Graph
    g = Graph()
    x = orc.randn(seed, shape)
    w = orc.randn(seed + 1, (co, shape[1], k, k), std=0.05)
    b = orc.randn(seed + 2, (co,), std=0.1)
    X = g.leaf(dev_tensor(x, io))
    Wt = g.leaf(dev_tensor(w, torch.float32))
    u = g.upscale(X, up) if up else X
    c = g.conv_2d_direct(Wt, u, p0=(k - 1) // 2, p1=(k - 1) // 2)
    y = g.add(c, g.reshape(g.leaf(dev_tensor(b, torch.float32)), [1, 1, co, 1])) if bias else c
    return g, (x, w, b), u, c, y


@pytest.mark.parametrize("io", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape,co,k,up", [((1, 24, 9, 20), 40, 3, 2), ((2, 16, 7, 5), 8, 1, 2),
                                           ((1, 64, 16, 24), 128, 3, None)])
def test_graph_conv2d_bias_upscale(orc, be, shape, co, k, up, io):
    """Conv2d::forward's CONV_2D_DIRECT + bias ADD, behind Upsample2D's
    nearest 2x UPSCALE: one convolution (weights packed, channel-last copy,
    conv) with the bias and the upsample folded in."""
    print(f"graph conv x={shape} co={co} k={k} up={up} {io}", flush=True)
    g, (x, w, b), u, c, y = _graph_conv(orc, io, shape, co, k, up)
    kernels, fused = g.compute(be, outputs=[y])
    torch.cuda.synchronize()
    # pack, channel-last copy (3x3, and 1x1 on bf16), conv
    assert fused == (2 if up else 1) and kernels == (3 if k == 3 or io == torch.bfloat16 else 2), (kernels, fused)
    ref = orc.conv2d(orc.round_bf16(as_input(x, io)), orc.round_bf16(w), b, up2=bool(up))
    check(host(y.torch()), ref, io, f"graph conv {shape}")


@pytest.mark.parametrize("io", [torch.float32, torch.bfloat16])
def test_graph_upscale_kept_and_factor_3(orc, be, io):
    """An UPSCALE that is itself an output runs the nearest-neighbour kernel
    (bit-exact repeat); the conv then reads it like any input.  Factor 3 is
    never folded into the conv."""
    for f in (2, 3):
        g, (x, w, b), u, c, y = _graph_conv(orc, io, (1, 16, 5, 7), 24, 3, f, seed=SEED + 330)
        kernels, fused = g.compute(be, outputs=[y, u])
        torch.cuda.synchronize()
        assert fused == 1 and kernels == 4, (f, kernels, fused)
        xs = as_input(x, io)
        up = np.repeat(np.repeat(xs, f, axis=2), f, axis=3)
        assert np.array_equal(host(u.torch()), up), f"upscale x{f}"
        ref = orc.conv2d(orc.round_bf16(up), orc.round_bf16(w), b)
        check(host(y.torch()), ref, io, f"conv after upscale x{f}")


def test_graph_conv_then_groupnorm_silu(orc, be):
    """A decoder resnet step: conv (+bias) -> GroupNorm(32) + SiLU; the conv
    output stays a real tensor between the two fused launches."""
    from graphkit import Graph
    io, N, Ci, Co, H, W, G = torch.bfloat16, 1, 32, 64, 12, 16, 32
    g, (x, w, b), u, c, y = _graph_conv(orc, io, (N, Ci, H, W), Co, 3, None, seed=SEED + 340)
    gw = orc.randn(SEED + 345, (Co,), mean=1.0, std=0.1)
    gb = orc.randn(SEED + 346, (Co,), std=0.1)
    v = g.reshape(y, [Co // G * H * W, G, N])
    r = g.reshape(g.norm(v, 1e-6), [W, H, Co, N])
    a = g.add(g.mul(r, g.leaf(dev_tensor(gw.reshape(1, Co, 1, 1), torch.float32))),
              g.leaf(dev_tensor(gb.reshape(1, Co, 1, 1), torch.float32)))
    out = g.mul(a, g.sigmoid(a))
    kernels, fused = g.compute(be, outputs=[out])
    torch.cuda.synchronize()
    assert kernels == 3 + 2, kernels
    conv_out = host(y.torch())
    check(conv_out, orc.conv2d(orc.round_bf16(x), orc.round_bf16(w), b), io, "conv")
    check(host(out.torch()), orc.groupnorm_silu(conv_out, G, gw, gb, 1e-6), io, "GroupNorm+SiLU after conv")


def test_graph_conv_rejects_stride_2(dev, be):
    from graphkit import Graph
    import dit_hip as dh
    g = Graph()
    X = g.leaf(torch.zeros((1, 4, 8, 8), dtype=torch.float32, device="cuda"))
    Wt = g.leaf(torch.zeros((4, 4, 3, 3), dtype=torch.float32, device="cuda"))
    y = g.conv_2d_direct(Wt, X, s0=2, s1=2)
    with pytest.raises(dh.DtError, match="stride 2,2"):
        g.compute(be, outputs=[y])


# ------------------------------------------------- residual epilogue (graph) --
# ResnetBlock2D's `(input + hidden) / output_scale_factor` (ResnetBlock2D.inl:194)
# records ADD(res, conv2 + bias) then SCALE; the executor runs both in conv2's
# epilogue with the ADD's value rounded where the graph stores it.

def _residual_graph(x, w, b, res, scale, io, alias):
    from graphkit import Graph
    g = Graph()
    Co, K = w.shape[0], w.shape[-1]
    X = g.leaf(dev_tensor(x, io))
    Wt = g.leaf(dev_tensor(w, torch.float32))
    B = g.leaf(dev_tensor(b, torch.float32))
    R = g.leaf(dev_tensor(res, io))
    c = g.conv_2d_direct(Wt, X, p0=K // 2, p1=K // 2)
    h = g.add(c, g.reshape(B, [1, 1, Co, 1]))
    y = g.scale(g.add(R, h), scale)
    if alias:      # the output in place over the residual, as an allocator may place it
        y.d.data = R.d.data
    return g, h, y, (R.data if alias else y.data)


@pytest.mark.parametrize("io", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape,co,k,scale,alias", [((1, 24, 9, 13), 40, 3, 0.5, False),
                                                    ((1, 64, 16, 20), 64, 3, 1.0, True),
                                                    ((2, 32, 7, 70), 48, 1, 1.0 / 3.0, False),
                                                    ((1, 128, 32, 32), 128, 3, 0.7, True),
                                                    ((4, 16, 256, 256), 24, 3, 0.5, True)])  # a batch, in place
def test_conv_residual_epilogue_equals_the_nodes(orc, dev, io, shape, co, k, scale, alias):
    """The fused conv + bias + ADD + SCALE launch stores the bits the nodes
    store when run one by one (conv + bias, ADD, SCALE: conv2's output kept
    as a graph output), in place over the residual or not, and matches
    the oracle's (res + conv(x) + b) * scale."""
    from graphkit import Backend
    print(f"conv residual x={shape} co={co} k={k} scale={scale} alias={alias} {io}", flush=True)
    x = orc.randn(SEED + 60, shape)
    w = orc.randn(SEED + 61, (co, shape[1], k, k), std=0.1)
    b = orc.randn(SEED + 62, (co,), std=0.1)
    res = orc.randn(SEED + 63, (shape[0], co, shape[2], shape[3]))
    be = Backend()
    try:
        g, h, y, out = _residual_graph(x, w, b, res, scale, io, alias)
        kernels, fused = g.compute(be.h, outputs=[y])
        torch.cuda.synchronize()
        fused_out = out.clone()
        g2, h2, y2, out2 = _residual_graph(x, w, b, res, scale, io, alias)
        kernels2, fused2 = g2.compute(be.h, outputs=[y2, h2])
        torch.cuda.synchronize()
    finally:
        be.close()
    # pack, channel-last copy (3x3, and 1x1 on bf16), conv
    assert (kernels, fused) == ((3 if k == 3 or io == torch.bfloat16 else 2), 3), (kernels, fused)
    assert (kernels2, fused2) == (kernels + 2, 1), (kernels2, fused2)
    assert torch.equal(fused_out.view(torch.int16 if io == torch.bfloat16 else torch.int32),
                       out2.view(torch.int16 if io == torch.bfloat16 else torch.int32))
    conv = orc.conv2d(orc.round_bf16(as_input(x, io)), orc.round_bf16(w), b)
    want = (as_input(res, io) + conv) * np.float32(scale)
    check(host(fused_out), want, io, "conv + residual", one_rounding=False)


# ----------------------------------------- GroupNorm in the channel-last copy --
# norm -> SiLU -> conv (ResnetBlock2D.inl:114-127, 163-176): the executor
# applies the GroupNorm (+ affine) (+ SiLU) as the 3x3 conv's channel-last
# copy reads its input, so the normalised tensor is never stored.

def _gn_conv_graph(x, gw, gb, G, w, b, io, affine, silu, up, res=None):
    from graphkit import Graph
    g = Graph()
    N, C, H, W = x.shape
    Co, K = w.shape[0], w.shape[-1]
    X = g.leaf(dev_tensor(x, io))
    v = g.reshape(X, [C // G * H * W, G, N])
    cur = g.reshape(g.norm(v, 1e-6), [W, H, C, N])
    if affine:
        cur = g.mul(cur, g.leaf(dev_tensor(gw.reshape(1, C, 1, 1), torch.float32)))
        cur = g.add(cur, g.leaf(dev_tensor(gb.reshape(1, C, 1, 1), torch.float32)))
    if silu:
        cur = g.mul(cur, g.sigmoid(cur))
    gn = cur
    u = g.upscale(gn, 2) if up else gn
    c = g.conv_2d_direct(g.leaf(dev_tensor(w, torch.float32)), u, p0=K // 2, p1=K // 2)
    y = g.add(c, g.reshape(g.leaf(dev_tensor(b, torch.float32)), [1, 1, Co, 1]))
    if res is not None:
        y = g.scale(g.add(g.leaf(dev_tensor(res, io)), y), 0.5)
    return g, gn, y


@pytest.mark.parametrize("io", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape,G,co,affine,silu,up,residual", [
    ((1, 64, 16, 24), 32, 64, True, True, False, False),
    ((2, 32, 9, 13), 8, 48, True, True, False, True),      # plane not a multiple of 8: scalar statistics
    ((1, 128, 32, 32), 32, 128, False, True, False, True),
    ((1, 48, 12, 20), 4, 40, True, False, True, False),    # no SiLU, 2x upscale between norm and conv
    ((1, 256, 20, 20), 32, 64, True, True, False, False)])
def test_groupnorm_folded_into_conv_equals_the_nodes(orc, dev, io, shape, G, co, affine, silu, up, residual):
    """Fused (GroupNorm statistics, (mean, rstd), the normalising
    channel-last copy, the conv) against the same nodes with the GroupNorm
    output kept as a graph output (two-pass GroupNorm, then the conv): the
    same bits; and against the oracle."""
    from graphkit import Backend
    print(f"gn+conv x={shape} G={G} co={co} affine={affine} silu={silu} up={up} res={residual} {io}", flush=True)
    x = orc.randn(SEED + 70, shape)
    gw = orc.randn(SEED + 71, (shape[1],), mean=1.0, std=0.1)
    gb = orc.randn(SEED + 72, (shape[1],), std=0.1)
    w = orc.randn(SEED + 73, (co, shape[1], 3, 3), std=0.05)
    b = orc.randn(SEED + 74, (co,), std=0.1)
    f = 2 if up else 1
    res = orc.randn(SEED + 75, (shape[0], co, shape[2] * f, shape[3] * f)) if residual else None
    be = Backend()
    try:
        g, gn, y = _gn_conv_graph(x, gw, gb, G, w, b, io, affine, silu, up, res)
        kernels, fused = g.compute(be.h, outputs=[y])
        torch.cuda.synchronize()
        fused_out = y.data.clone()
        g2, gn2, y2 = _gn_conv_graph(x, gw, gb, G, w, b, io, affine, silu, up, res)
        kernels2, fused2 = g2.compute(be.h, outputs=[y2, gn2])
        torch.cuda.synchronize()
        gn_out = gn2.data.clone()
    finally:
        be.close()
    # statistics + (mean, rstd) replace statistics + apply (then pack, copy, conv): the same
    # five launches, and the GroupNorm's root joins the conv's plan
    assert kernels == kernels2 == 5 and fused == fused2 + 1, (kernels, kernels2, fused, fused2)
    bits = torch.int16 if io == torch.bfloat16 else torch.int32
    assert torch.equal(fused_out.view(bits), y2.data.view(bits))
    ref_gn = orc.groupnorm_silu(as_input(x, io), G, gw if affine else None, gb if affine else None, 1e-6, silu=silu)
    check(host(gn_out), ref_gn, io, "GroupNorm (unfused)", one_rounding=False)
    want = orc.conv2d(orc.round_bf16(host(gn_out)), orc.round_bf16(w), b, up2=up)
    if residual:
        want = (as_input(res, io) + want) * np.float32(0.5)
    check(host(fused_out), want, io, "GroupNorm + conv", one_rounding=False)


# 512-pixel tiles (16 x 32) are taken when they still give two workgroups
# per CU (N x tiles x output-channel tiles >= 512); these shapes reach them,
# with a batch, a partial output-channel tile, a partial column tile and the
# 2x upscale.
@pytest.mark.parametrize("io", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape,co,up2", [((4, 16, 256, 256), 24, False), ((1, 8, 512, 520), 16, False),
                                          ((1, 16, 256, 256), 8, True)])
def test_conv2d_512_pixel_tiles(orc, dev, shape, co, up2, io):
    print(f"conv2d 512px x={shape} co={co} up2={up2} {io}", flush=True)
    x = orc.randn(SEED + 90, shape)
    w = orc.randn(SEED + 91, (co, shape[1], 3, 3), std=0.2)
    b = orc.randn(SEED + 92, (co,), std=0.1)
    wp = dit_hip.conv2d_pack(dev_tensor(w, torch.float32))
    y = dit_hip.conv2d(dev_tensor(x, io), wp, bias=dev_tensor(b, torch.float32), upscale2=up2, workspace=True)
    torch.cuda.synchronize()
    ref = orc.conv2d(orc.round_bf16(as_input(x, io)), orc.round_bf16(w), b, up2=up2)
    check(host(y), ref, io, f"conv2d 512px {shape} -> {co}")
