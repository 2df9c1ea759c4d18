"""Pins the oracle (CPU restatement of the ggml ops) before anything is
checked against it: known-answer vectors, the golden fixtures written by
tests/golden/make_golden.py from library routines and byte-level format
packers, closed forms, invariants and brute force on tiny inputs.  Each
check is chosen so that a plausible restatement mistake (dropped term, wrong
sign, wrong index, transposed operand) fails it."""
import json
import os

import numpy as np
import pytest
import torch

from conftest import assert_fp32

GOLD = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def fx():
    with np.load(os.path.join(GOLD, "chain_golden.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="module")
def qkat():
    with open(os.path.join(GOLD, "quant_kat.json")) as f:
        return json.load(f)


# ---- generator ------------------------------------------------------------

def test_mt19937_64_known_answer(orc):
    # The C++ standard fixes the 10000th output of a default-seeded mt19937_64.
    assert orc.mt64_nth(5489, 10000) == 9981545732273789042


def test_hash_primitives_known_answers(orc):
    """splitmix64's published first outputs for seed 0 (Vigna's splitmix64.c:
    output n = mix(n * 0x9E3779B97F4A7C15)) and FNV-1a 64 test vectors."""
    lib, G = orc.load(), 0x9E3779B97F4A7C15
    assert lib.or_splitmix64(G) == 0xE220A8397B1DCDAF
    assert lib.or_splitmix64((2 * G) % 2**64) == 0x6E789E6AA1B965F4
    assert lib.or_splitmix64((3 * G) % 2**64) == 0x06C45D188009454F
    assert lib.or_fnv1a64(b"") == 0xCBF29CE484222325
    assert lib.or_fnv1a64(b"a") == 0xAF63DC4C8601EC8C
    assert lib.or_fnv1a64(b"foobar") == 0x85944171F73967E8
    assert orc.hash_key(7, "w") == lib.or_splitmix64((7 * G % 2**64) ^ lib.or_fnv1a64(b"w"))


def test_hash_q8_0_weights(orc):
    """The hash-drawn Q8_0 rule (dit_cli --hash-weights): block b takes
    z(9b) for its fp16 scale and z(9b+1..8) for its codes, composed here from
    the pinned primitives for a few blocks; codes stay in [-127, 127] with the
    triangular law's spread (std 255/(2 sqrt 6) ~ 52.1), the scale in
    [0x0E00, 0x0FFF]; another path or seed changes every block."""
    lib, G = orc.load(), 0x9E3779B97F4A7C15
    rows, cols = 96, 256
    b = orc.hash_q8_0(3, "blocks.0.w", rows, cols).reshape(-1, 34)
    key = orc.hash_key(3, "blocks.0.w")
    z = lambda i: lib.or_splitmix64((key + i * G) % 2**64)
    for blk in (0, 1, 5, rows * cols // 32 - 1):
        d = z(9 * blk) & 0x1FF | 0x0E00
        assert int(b[blk, 0]) | int(b[blk, 1]) << 8 == d
        for k in range(1, 9):
            y = [(z(9 * blk + k) >> (8 * j)) & 0xFF for j in range(8)]
            for m in range(4):
                q = int((y[2 * m] + y[2 * m + 1] - 255) / 2)  # truncation toward zero
                assert np.int8(b[blk, 2 + 4 * (k - 1) + m].view(np.int8)) == q
    codes = b[:, 2:].view(np.int8).astype(np.float64)
    assert codes.min() >= -127 and codes.max() <= 127
    assert abs(codes.std() - 255 / (2 * np.sqrt(6))) < 1.0 and abs(codes.mean()) < 1.0
    dbits = b[:, 0].astype(np.int64) | b[:, 1].astype(np.int64) << 8
    assert dbits.min() >= 0x0E00 and dbits.max() <= 0x0FFF
    other = orc.hash_q8_0(3, "blocks.1.w", rows, cols).reshape(-1, 34)
    assert (other != b).any(axis=1).all()
    assert (orc.hash_q8_0(4, "blocks.0.w", rows, cols).reshape(-1, 34) != b).any(axis=1).all()
    w = orc.dequantize(b.ravel(), rows * cols, 8)
    assert 0.018 < w.std() < 0.026


def test_hash_norm_weights(orc):
    """RMSNorm weights of the rule: 1 + (top 24 bits of z(i) - 2^23) * 2^-28,
    within 2^-5 of 1, element i from z(i)."""
    lib, G = orc.load(), 0x9E3779B97F4A7C15
    w = orc.hash_norm_weight(9, "attn.norm_q.weight", 128)
    key = orc.hash_key(9, "attn.norm_q.weight")
    for i in (0, 1, 127):
        v = (lib.or_splitmix64((key + i * G) % 2**64) >> 40) - (1 << 23)
        assert w[i] == np.float32(1.0) + np.float32(v * 2.0**-28)
    assert np.all(np.abs(w - 1) <= 2.0**-5) and w.std() > 0.005


def test_randn_is_standard_normal(orc):
    from scipy import stats
    x = orc.randn(orc.tensor_seed(0), (200_000,)).astype(np.float64)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    assert stats.kstest(x, "norm").pvalue > 1e-3
    y = orc.randn(orc.tensor_seed(1), (1000,), mean=1.0, std=0.02).astype(np.float64)
    assert abs(y.mean() - 1.0) < 0.005 and abs(y.std() - 0.02) < 0.003
    # Seeds are independent streams; the same seed is reproducible.
    assert not np.array_equal(orc.randn(5, (8,)), orc.randn(6, (8,)))
    assert np.array_equal(orc.randn(5, (9,)), orc.randn(5, (9,)))


# ---- number formats -----------------------------------------------------------

def test_f16_decode_exhaustive(orc):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(want)]))


def test_f16_encode_matches_numpy_rne(orc):
    rng = np.random.RandomState(3)
    vals = np.concatenate([
        rng.randn(3000).astype(np.float32) * np.float32(100),
        rng.randn(2000).astype(np.float32) * np.float32(1e-6),   # subnormal range
        np.array([65504, 65519.99, 65520, 65536, 1e9, 2 ** -24, 2 ** -25, 3 * 2 ** -26,
                  2 ** -25 * 1.0000001, 6.1e-5, -0.0, 0.0], dtype=np.float32),
        # exact halfway points between neighbouring fp16 values
        (np.arange(1, 4000, dtype=np.float32) * np.float32(2 ** -11) + np.float32(2 ** -12)),
    ])
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    got = np.array([orc.f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, want)


def test_bf16_matches_torch_rne(orc, fx):
    assert np.array_equal(orc.to_bf16_bits(fx["bf16_in"]), fx["bf16_bits"])
    back = orc.from_bf16_bits(fx["bf16_bits"])
    assert np.array_equal(back, torch.from_numpy(fx["bf16_bits"].view(np.int16)).view(
        torch.bfloat16).float().numpy())


# ---- norms / activations ------------------------------------------------------

@pytest.mark.parametrize("name", ["ln_small", "ln_3072"])
def test_norm_and_adaln_vs_torch(orc, fx, name):
    x = fx[name + "_x"]
    assert_fp32(orc.norm(x, 1e-6), fx[name + "_norm"], what="norm")
    assert_fp32(orc.adaln(x, fx[name + "_shift"], fx[name + "_scale"], 1e-6),
                fx[name + "_adaln"], what="adaln")


def test_norm_invariants(orc):
    x = orc.randn(11, (7, 257)) * 3 + 5
    y = orc.norm(x, 1e-6).astype(np.float64)
    assert np.allclose(y.mean(-1), 0, atol=1e-5) and np.allclose(y.var(-1), 1, atol=1e-4)
    # shift / scale invariance of the normalisation
    assert_fp32(orc.norm(x * 4 - 3, 1e-6), orc.norm(x, 1e-6), tol=2e-5, what="equivariance")
    # constant rows normalise to zero
    assert np.all(orc.norm(np.full((2, 64), 3.25, np.float32), 1e-6) == 0)


@pytest.mark.parametrize("name", ["rms_small", "rms_128"])
def test_rms_norm_vs_torch(orc, fx, name):
    x, w = fx[name + "_x"], fx[name + "_w"]
    got = orc.binary(2, orc.rms_norm(x, 1e-6), w)
    assert_fp32(got, fx[name + "_y"], what="rms_norm*w")


def test_sigmoid_and_swiglu_vs_torch(orc, fx):
    assert_fp32(orc.sigmoid(fx["act_g"]), fx["act_sigmoid"], what="sigmoid")
    assert_fp32(orc.swiglu(fx["act_g"][None], fx["act_u"][None])[0], fx["act_swiglu"], what="swiglu")


def test_gated_residual_and_euler_closed_form(orc):
    h = orc.randn(1, (5, 48))
    o = orc.randn(2, (5, 48))
    g = orc.randn(3, (48,))
    want = h.astype(np.float64) + o.astype(np.float64) * g.astype(np.float64)
    assert_fp32(orc.gated_residual(h, o, g), want, what="gated")
    assert_fp32(orc.euler(h, o, 0.125), h + o.astype(np.float64) * 0.125, what="euler")


@pytest.mark.parametrize("name,G", [("gn_a", 2), ("gn_b", 4), ("gn_c", 32)])
def test_groupnorm_silu_vs_torch(orc, fx, name, G):
    x, w, b = fx[name + "_x"], fx[name + "_w"], fx[name + "_b"]
    assert_fp32(orc.groupnorm_silu(x, G, w, b, 1e-6, silu=False), fx[name + "_gn"], what="gn")
    assert_fp32(orc.groupnorm_silu(x, G, w, b, 1e-6, silu=True), fx[name + "_silu"], what="gn+silu")
    # no affine == torch with unit weight / zero bias
    ref = torch.nn.functional.group_norm(torch.from_numpy(x.astype(np.float64)), G, eps=1e-6)
    assert_fp32(orc.groupnorm_silu(x, G, None, None, 1e-6, silu=False), ref.numpy(), what="gn noaff")


# ---- broadcast / concat -------------------------------------------------------

def test_binary_broadcast_is_modulo_repeat(orc):
    a = orc.randn(4, (2, 3, 4, 6))
    for bshape in [(6,), (1, 1, 1, 6), (1, 3, 1, 6), (2, 1, 4, 1), (1, 1, 2, 3), (2, 3, 4, 6)]:
        b = orc.randn(5, bshape)
        b4 = b.reshape((1,) * (4 - b.ndim) + b.shape)
        reps = [a.shape[i] // b4.shape[i] for i in range(4)]
        tiled = np.tile(b4, reps).astype(np.float64)
        for op, f in ((0, np.add), (1, np.subtract), (2, np.multiply), (3, np.divide)):
            assert_fp32(orc.binary(op, a, b), f(a.astype(np.float64), tiled), what=f"op{op} {bshape}")
    # strided (transposed) src0 view
    at = a.transpose(0, 1, 3, 2)
    assert_fp32(orc.binary(0, at, np.float32(1.0) * np.ones(4, np.float32)), at + 1.0, what="strided")


def test_concat_matches_numpy(orc):
    a, b = orc.randn(6, (2, 3, 4)), orc.randn(7, (2, 3, 5))
    assert np.array_equal(orc.concat(a, b, 0), np.concatenate([a, b], -1))
    c = orc.randn(8, (2, 5, 4))
    assert np.array_equal(orc.concat(a, c[:, :3] * 0 + c[:, 2:5], 1), np.concatenate([a, c[:, 2:5]], 1))


# ---- RoPE -----------------------------------------------------------------------

def test_rope_cache_recurrence(orc):
    # theta_i = p * base^(-2i/d) up to the fp32 recurrence drift (<= 16 ulps of
    # the angle at pair 15), and cos/sin of exactly that angle.
    for p in (0, 1, 7, 63, 511):
        c = orc.rope_cache(float(p), 32, 32, 10000.0).astype(np.float64)
        th = p * 10000.0 ** (-np.arange(0, 32, 2) / 32.0)
        assert np.allclose(c[0::2], np.cos(th), atol=4e-6 * max(p, 1) + 1e-7)
        assert np.allclose(c[1::2], np.sin(th), atol=4e-6 * max(p, 1) + 1e-7)
    # p = 0 is the identity rotation
    c0 = orc.rope_cache(0.0, 32, 32, 10000.0)
    assert np.all(c0[0::2] == 1) and np.all(c0[1::2] == 0)


@pytest.mark.parametrize("case,axes,theta,tol", [("rope_toy", [2] * 4, 10000, 1e-5),
                                                 ("rope_flux", [32] * 4, 2000, 1e-5),
                                                 ("rope_far", [32] * 4, 10000, 2e-3)])
def test_rope_vs_diffusers_complex_form(orc, fx, case, axes, theta, tol):
    x, pos, want = fx[case + "_x"], fx[case + "_pos"], fx[case + "_y"]
    # rope_ext per axis section + concat, as Flux2PosEmbed emits it
    out, off = [], 0
    for a, d in enumerate(axes):
        out.append(orc.rope_normal(x[None, :, :, off:off + d], pos[:, a], d, float(theta))[0])
        off += d
    got = np.concatenate(out, -1)
    assert_fp32(got, want, tol=tol, what=case)


def test_qk_rmsnorm_rope_chain(orc, fx):
    x, pos = fx["rope_flux_x"], fx["rope_flux_pos"]
    w = orc.randn(9, (128,), mean=1.0, std=0.02)
    xt = torch.from_numpy(x.astype(np.float64))
    z = (torch.nn.functional.rms_norm(xt, (128,), eps=1e-6) * torch.from_numpy(w.astype(np.float64))).numpy()
    # float64 complex rotation (diffusers' apply_rotary_emb form), theta 2000
    from numpy import exp
    want = np.empty_like(z)
    for a in range(4):
        d, off = 32, 32 * a
        fr = 1.0 / (2000.0 ** (np.arange(0, d, 2) / d))
        ang = pos[:, a][:, None] * fr[None]
        zz = z[..., off:off + d:2] + 1j * z[..., off + 1:off + d:2]
        r = zz * exp(1j * ang)[:, None, :]
        want[..., off:off + d:2], want[..., off + 1:off + d:2] = r.real, r.imag
    got = orc.qk_rmsnorm_rope(x, w, pos, 32, 2000.0, 1e-6)
    assert_fp32(got, want, what="qk chain")
    # invariant: all-zero positions leave the normalised vector unrotated
    got0 = orc.qk_rmsnorm_rope(x, w, np.zeros_like(pos), 32, 2000.0, 1e-6)
    assert_fp32(got0, z, what="p=0")
    # one non-zero axis changes only that axis' 32 dims
    p1 = np.zeros_like(pos)
    p1[:, 2] = 5
    g1 = orc.qk_rmsnorm_rope(x, w, p1, 32, 2000.0, 1e-6)
    assert np.array_equal(g1[..., :64], got0[..., :64]) and np.array_equal(g1[..., 96:], got0[..., 96:])
    assert not np.array_equal(g1[..., 64:96], got0[..., 64:96])


# ---- quantisation ---------------------------------------------------------------

def test_q8_0_known_answers(orc, qkat):
    for case in qkat["q8_0"]:
        blk = np.frombuffer(bytes.fromhex(case["block"]), dtype=np.uint8)
        got = orc.dequantize(blk, 32, 8)
        assert np.array_equal(got.view(np.uint32), np.array(case["expected_f32_bits"], np.uint32))


def test_q4_K_known_answers(orc, qkat):
    for case in qkat["q4_K"]:
        blk = np.frombuffer(bytes.fromhex(case["block"]), dtype=np.uint8)
        # 6-bit scale/min unpack of every sub-block
        for j in range(8):
            assert orc.q4_K_scale_min(j, blk[4:16]) == (case["sc"][j], case["m"][j])
        got = orc.dequantize(blk, 256, 12)
        assert np.array_equal(got.view(np.uint32), np.array(case["expected_f32_bits"], np.uint32))


@pytest.mark.parametrize("qtype,qk", [(8, 32), (12, 256)])
def test_quantizer_round_trip(orc, qtype, qk):
    w = orc.randn(orc.tensor_seed(40), (8, 1024), std=0.02)
    b = orc.quantize(w, qtype)
    assert b.size == w.size // qk * (34 if qtype == 8 else 144)
    y = orc.dequantize(b, w.size, qtype).reshape(w.shape)
    blocks = np.abs(w).reshape(-1, qk).max(1)
    err = np.abs(y - w).reshape(-1, qk).max(1)
    # Q8_0: codes come from the fp32 step d = amax/127 but d is stored as fp16,
    # so error <= d/2 + 127 * |d - fp16(d)| <= d * (0.5 + 127 * 2^-11).
    # Q4_K: within ~1/15 of the block range.
    bound = blocks / 127 * (0.5 + 127 * 2.0 ** -11) * 1.001 + 1e-9 if qtype == 8 \
        else blocks * 2 / 15 * 0.75
    assert np.all(err <= bound)
    if qtype == 8:
        # codes reach +-127 in every block (amax maps to the top code)
        q = b.reshape(-1, 34)[:, 2:].view(np.int8)
        assert np.all(np.abs(q).max(1) == 127)


# ---- matmul and attention ---------------------------------------------------

@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (3, 5, 7), (37, 45, 130), (64, 64, 256), (5, 9, 3)])
def test_linear_vs_torch_float64(orc, M, N, K):
    """Blocked 2x4 path, scalar tails and K % 4 != 0 all against float64."""
    x = orc.randn(orc.tensor_seed(50), (M, K))
    w = orc.randn(orc.tensor_seed(51), (N, K), std=0.02)
    b = orc.randn(orc.tensor_seed(52), (N,))
    ref = torch.from_numpy(x).double() @ torch.from_numpy(w).double().T
    assert_fp32(orc.linear(x, w), ref.numpy(), tol=1e-6, what="linear")
    assert_fp32(orc.linear(x, w, b), (ref + torch.from_numpy(b).double()).numpy(), tol=1e-6,
                what="linear+bias")


def test_linear_q8_0_ggml_brute_force(orc):
    """ggml's Q8_0 mul_mat arithmetic: activation rows quantised to Q8_0,
    exact integer block dots, each block term (float)dot * (d_x * d_w) and the
    running sum in fp32 -- here spelled out per element in numpy from the
    quantiser's bytes, with a bias; bit-identical."""
    M, N, K = 7, 5, 96
    x = orc.randn(orc.tensor_seed(56), (M, K))
    w = orc.randn(orc.tensor_seed(57), (N, K), std=0.02)
    b = orc.randn(orc.tensor_seed(58), (N,))
    W = orc.Q8_0Weight(orc.quantize(w, 8), N, K)
    qx = orc.quantize(x, 8).reshape(M, K // 32, 34)
    qw = W.blocks.reshape(N, K // 32, 34)
    f32 = np.float32
    want = np.empty((M, N), np.float32)
    for i in range(M):
        for j in range(N):
            s = f32(0)
            for c in range(K // 32):
                dot = int((qx[i, c, 2:].view(np.int8).astype(np.int64) * qw[j, c, 2:].view(np.int8)).sum())
                d = f32(qx[i, c, :2].view(np.float16)[0]) * f32(qw[j, c, :2].view(np.float16)[0])
                s = f32(s + f32(f32(dot) * d))
            want[i, j] = f32(s + b[j])
    assert np.array_equal(orc.linear(x, W, b), want)


def test_linear_q8_0_ggml_invariants(orc):
    """Activations that Q8_0 represents exactly (each block's amax 127 d, d an
    fp16 value, every element d q) requantise losslessly, so the product is
    the exact one (fp32 summation order aside); a Gaussian activation's
    quantisation error sits at the Q8_0 level (relative L2 ~ 1/(127 sqrt 12)
    of the block amax per element, 0.3-1% of the output here)."""
    M, N, K = 9, 40, 256
    rng = np.random.default_rng(5)
    d = rng.integers(0x2000, 0x3C00, (M, K // 32)).astype(np.uint16).view(np.float16).astype(np.float32)
    q = rng.integers(-127, 128, (M, K // 32, 32))
    q[:, :, 0] = 127
    x = (d[:, :, None] * q).reshape(M, K).astype(np.float32)
    w = orc.randn(orc.tensor_seed(59), (N, K), std=0.02)
    W = orc.Q8_0Weight(orc.quantize(w, 8), N, K)
    wd = W.dequantize()
    exact = x.astype(np.float64) @ wd.astype(np.float64).T
    assert_fp32(orc.linear(x, W), exact, tol=2e-6, what="q8_0 ggml on representable activations")
    g = orc.randn(orc.tensor_seed(60), (M, K))
    rel = np.linalg.norm(orc.linear(g, W) - orc.linear(g, wd)) / np.linalg.norm(orc.linear(g, wd))
    assert 2e-3 < rel < 1.5e-2, rel


def test_linear_operand_roles(orc):
    """y = x W^T, not x W or W x: a rectangular identity-like W picks columns."""
    x = orc.randn(orc.tensor_seed(53), (6, 8))
    w = np.zeros((3, 8), np.float32)
    w[0, 2] = w[1, 7] = w[2, 0] = 1.0
    assert np.array_equal(orc.linear(x, w), x[:, [2, 7, 0]])


@pytest.mark.parametrize("Sq,Skv,H,D", [(1, 1, 1, 4), (7, 5, 2, 16), (70, 50, 3, 128)])
def test_attention_vs_torch_sdpa(orc, Sq, Skv, H, D):
    q = orc.randn(orc.tensor_seed(54), (Sq, H, D))
    k = orc.randn(orc.tensor_seed(55), (Skv, H, D))
    v = orc.randn(orc.tensor_seed(56), (Skv, H, D))
    t = lambda a: torch.from_numpy(a).double().transpose(0, 1)
    ref = torch.nn.functional.scaled_dot_product_attention(t(q), t(k), t(v)).transpose(0, 1).numpy()
    assert_fp32(orc.attention(q, k, v), ref, tol=1e-6, what="attention")


def test_attention_closed_forms(orc):
    """One key returns its value row; scale 0 averages V; a dominant score
    selects its key (checks which operand is softmaxed over which axis)."""
    q = orc.randn(orc.tensor_seed(57), (9, 2, 8))
    v1 = orc.randn(orc.tensor_seed(58), (1, 2, 8))
    k1 = orc.randn(orc.tensor_seed(59), (1, 2, 8))
    assert np.allclose(orc.attention(q, k1, v1), np.broadcast_to(v1, q.shape), atol=1e-7)
    k = orc.randn(orc.tensor_seed(60), (11, 2, 8))
    v = orc.randn(orc.tensor_seed(61), (11, 2, 8))
    assert np.allclose(orc.attention(q, k, v, scale=0.0), np.broadcast_to(v.mean(0), q.shape), atol=1e-6)
    kd = np.zeros((11, 2, 8), np.float32)
    kd[4] = 1.0
    qd = np.ones((3, 2, 8), np.float32)
    out = orc.attention(qd, kd, v, scale=100.0)
    assert np.allclose(out, np.broadcast_to(v[4], out.shape), atol=1e-6)


# ------------------------------------------------------------------ conv2d --
@pytest.mark.parametrize("shape,co,k,up2", [((2, 5, 7, 9), 4, 3, False), ((1, 3, 6, 5), 2, 3, True),
                                            ((1, 6, 4, 4), 7, 1, False), ((1, 2, 3, 3), 3, 1, True)])
def test_conv2d_matches_torch(orc, shape, co, k, up2):
    """conv_2d_direct + bias (stride 1, padding (k-1)/2), optionally on the
    nearest 2x upscale, against torch's float64 conv2d."""
    torch = pytest.importorskip("torch")
    x = orc.randn(901, shape)
    w = orc.randn(902, (co, shape[1], k, k))
    b = orc.randn(903, (co,))
    y = orc.conv2d(x, w, b, up2=up2)
    xt = torch.from_numpy(x).double()
    if up2:
        xt = torch.nn.functional.interpolate(xt, scale_factor=2, mode="nearest")
    t = torch.nn.functional.conv2d(xt, torch.from_numpy(w).double(), torch.from_numpy(b).double(),
                                   padding=(k - 1) // 2).numpy()
    assert y.shape == t.shape
    assert np.abs(y - t).max() <= 1e-5 * max(1.0, np.abs(t).max())


def test_conv2d_closed_forms(orc):
    """A centre-tap kernel returns x (+ b) exactly; an all-ones kernel on
    ones counts the taps inside the image: 9 inside, 6 on an edge, 4 at a
    corner; the same on the upscale sees each source pixel twice per axis."""
    x = orc.randn(904, (1, 3, 5, 6))
    w = np.zeros((3, 3, 3, 3), np.float32)
    for c in range(3):
        w[c, c, 1, 1] = 1.0
    b = np.array([0.5, -1.0, 2.0], np.float32)
    assert np.array_equal(orc.conv2d(x, w, b), x + b[None, :, None, None])
    ones = np.ones((1, 1, 4, 5), np.float32)
    y = orc.conv2d(ones, np.ones((1, 1, 3, 3), np.float32))[0, 0]
    assert y[0, 0] == 4 and y[0, 2] == 6 and y[2, 0] == 6 and y[1, 1] == 9 and y[3, 4] == 4
    yu = orc.conv2d(np.arange(4, dtype=np.float32).reshape(1, 1, 2, 2), np.ones((1, 1, 1, 1), np.float32), up2=True)
    assert np.array_equal(yu[0, 0], np.array([[0, 0, 1, 1], [0, 0, 1, 1], [2, 2, 3, 3], [2, 2, 3, 3]], np.float32))
