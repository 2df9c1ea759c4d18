"""Writes the golden fixtures that pin the oracle, WITHOUT using the oracle.

Each expected output comes from a source independent of the oracle's code:
  * ggml block formats (Q8_0, Q4_K): blocks assembled byte by byte from
    chosen field values by the packers below (written from the published
    format description), expected values computed with numpy float32
    arithmetic (one IEEE rounding per operation, in the format's order);
  * norms / activations / RoPE: PyTorch library routines in float64
    (layer_norm, rms_norm, group_norm, sigmoid) and the diffusers-style
    complex rotation of Flux2PosEmbed restated in float64;
  * number formats: numpy float16 and torch bfloat16 conversions.
Shapes mirror the reference's own unit tests (test/src/nn/modules/
normalization/*.py, test/src/diffusers/models/transformers/flux2/
Flux2PosEmbed.py) plus a few Flux2-sized rows.

Run:  python tests/golden/make_golden.py   (rewrites the files next to it)
"""
import json
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
rng = np.random.RandomState(20251201)


def f16_bits(x):
    return int(np.array(x, dtype=np.float16).view(np.uint16))


# ---------------------------------------------------------------- Q8_0 --------
def q8_0_block(d_bits, qs):
    b = bytearray(34)
    b[0:2] = int(d_bits).to_bytes(2, "little")
    for j, q in enumerate(qs):
        b[2 + j] = q & 0xFF
    return bytes(b)


def q8_0_expected(d_bits, qs):
    d = np.array([d_bits], dtype=np.uint16).view(np.float16).astype(np.float32)[0]
    return [float(np.float32(d) * np.float32(q)) for q in qs]


q8_cases = []
for d_bits in [0x3C00, 0x0001, 0x03FF, 0x0400, 0x7BFF, 0xB800, 0x0000, 0x8000, 0x2E66, 0x1A3F]:
    qs = [(-128 + 8 * j) if j < 32 else 0 for j in range(32)]
    qs[31] = 127
    q8_cases.append((d_bits, qs))
for _ in range(6):
    d_bits = f16_bits(rng.uniform(1e-4, 0.1))
    qs = [int(v) for v in rng.randint(-128, 128, size=32)]
    q8_cases.append((d_bits, qs))
q8 = [{"block": q8_0_block(d, q).hex(), "expected_f32_bits":
       [int(np.float32(v).view(np.uint32)) for v in q8_0_expected(d, q)]} for d, q in q8_cases]


# ---------------------------------------------------------------- Q4_K --------
def pack_q4_k_scales(sc, mn):
    """12 bytes holding eight 6-bit scales and mins.  Sub-blocks 0-3 keep
    their low 6 bits in bytes 0-3 (scale) and 4-7 (min); sub-blocks 4-7 keep
    their low nibbles in bytes 8-11 (scale low, min high) and their top two
    bits in the top two bits of bytes 0-3 (scale) and 4-7 (min)."""
    out = [0] * 12
    for j in range(8):
        s, m = sc[j], mn[j]
        assert 0 <= s < 64 and 0 <= m < 64
        if j < 4:
            out[j] |= s
            out[4 + j] |= m
        else:
            out[8 + j - 4] |= (s & 0xF) | ((m & 0xF) << 4)
            out[j - 4] |= (s >> 4) << 6
            out[j] |= (m >> 4) << 6
    return bytes(out)


def q4_k_block(d_bits, dmin_bits, sc, mn, q):
    """q: 256 4-bit codes in element order.  Element 64c+l (l < 32) is the
    low nibble of qs[32c+l]; element 64c+32+l is its high nibble."""
    qs = bytearray(128)
    for c in range(4):
        for l in range(32):
            qs[32 * c + l] = (q[64 * c + l] & 0xF) | ((q[64 * c + 32 + l] & 0xF) << 4)
    return (int(d_bits).to_bytes(2, "little") + int(dmin_bits).to_bytes(2, "little")
            + pack_q4_k_scales(sc, mn) + bytes(qs))


def q4_k_expected(d_bits, dmin_bits, sc, mn, q):
    d = np.array([d_bits], dtype=np.uint16).view(np.float16).astype(np.float32)[0]
    dm = np.array([dmin_bits], dtype=np.uint16).view(np.float16).astype(np.float32)[0]
    out = []
    for e in range(256):
        j = e // 32            # sub-block of element e
        d1 = np.float32(d) * np.float32(sc[j])
        m1 = np.float32(dm) * np.float32(mn[j])
        out.append(float(np.float32(d1 * np.float32(q[e])) - m1))
    return out


q4_cases = []
# structured: distinct scale/min per sub-block, every code value present
q4_cases.append((0x3C00, 0x3800, [1, 2, 3, 4, 61, 62, 63, 17], [0, 5, 63, 33, 48, 16, 1, 62],
                 [e % 16 for e in range(256)]))
q4_cases.append((0x2E66, 0x2A00, [63] * 8, [63] * 8, [15 - (e % 16) for e in range(256)]))
q4_cases.append((0x0001, 0x03FF, [33, 17, 9, 5, 48, 40, 36, 34], [32, 16, 8, 4, 49, 41, 37, 35],
                 [(7 * e) % 16 for e in range(256)]))
for _ in range(5):
    q4_cases.append((f16_bits(rng.uniform(1e-4, 0.05)), f16_bits(rng.uniform(1e-4, 0.05)),
                     [int(v) for v in rng.randint(0, 64, 8)], [int(v) for v in rng.randint(0, 64, 8)],
                     [int(v) for v in rng.randint(0, 16, 256)]))
q4 = [{"block": q4_k_block(*c).hex(), "sc": c[2], "m": c[3],
       "expected_f32_bits": [int(np.float32(v).view(np.uint32)) for v in q4_k_expected(*c)]}
      for c in q4_cases]

with open(os.path.join(HERE, "quant_kat.json"), "w") as f:
    json.dump({"q8_0": q8, "q4_K": q4}, f, indent=0)


# ------------------------------------------------ norms / activations / RoPE --
def t64(a):
    return torch.from_numpy(np.asarray(a, dtype=np.float64))


fx = {}
# LayerNorm(3) on [2,2,3] (LayerNorm.py) and a Flux2-sized row batch, eps 1e-6.
for name, shape in (("ln_small", (2, 2, 3)), ("ln_3072", (3, 3072))):
    x = rng.randn(*shape).astype(np.float32)
    sh = (0.1 * rng.randn(shape[-1])).astype(np.float32)
    sc = (0.1 * rng.randn(shape[-1])).astype(np.float32)
    n = torch.nn.functional.layer_norm(t64(x), (shape[-1],), eps=1e-6).numpy()
    fx[name + "_x"], fx[name + "_shift"], fx[name + "_scale"] = x, sh, sc
    fx[name + "_norm"] = n
    fx[name + "_adaln"] = n * (1.0 + sc.astype(np.float64)) + sh.astype(np.float64)

# RMSNorm over heads of 128 and the toy dim 40 of the reference block tests.
for name, shape in (("rms_small", (4, 2, 40)), ("rms_128", (6, 24, 128))):
    x = rng.randn(*shape).astype(np.float32)
    w = (1.0 + 0.02 * rng.randn(shape[-1])).astype(np.float32)
    fx[name + "_x"], fx[name + "_w"] = x, w
    fx[name + "_y"] = (torch.nn.functional.rms_norm(t64(x), (shape[-1],), eps=1e-6) * t64(w)).numpy()

# GroupNorm(2, 4) on [2,4,3,3], GroupNorm(4, 8) on [1,8,4,4] (GroupNorm.py)
# and GroupNorm(32, 64) on [1,64,8,8], each followed by SiLU.
for name, (shape, G) in (("gn_a", ((2, 4, 3, 3), 2)), ("gn_b", ((1, 8, 4, 4), 4)),
                         ("gn_c", ((1, 64, 8, 8), 32))):
    x = rng.randn(*shape).astype(np.float32)
    w = (1.0 + 0.02 * rng.randn(shape[1])).astype(np.float32)
    b = (0.02 * rng.randn(shape[1])).astype(np.float32)
    gn = torch.nn.functional.group_norm(t64(x), G, t64(w), t64(b), eps=1e-6)
    fx[name + "_x"], fx[name + "_w"], fx[name + "_b"] = x, w, b
    fx[name + "_gn"] = gn.numpy()
    fx[name + "_silu"] = (gn * torch.sigmoid(gn)).numpy()

# SwiGLU / sigmoid on a spread of values.
g = np.concatenate([np.linspace(-30, 30, 241), rng.randn(271) * 4]).astype(np.float32)
u = rng.randn(g.size).astype(np.float32)
fx["act_g"], fx["act_u"] = g, u
fx["act_sigmoid"] = torch.sigmoid(t64(g)).numpy()
fx["act_swiglu"] = (t64(g) * torch.sigmoid(t64(g)) * t64(u)).numpy()


def rope_diffusers(x, pos, axes_dim, theta):
    """Flux2PosEmbed + apply_rotary_emb in float64: per axis a, frequencies
    theta^(-2i/d_a), angle = pos[:, a] * freq, adjacent pairs (x0, x1)
    rotated as the complex product (x0 + i x1) * e^(i angle)."""
    x = np.asarray(x, dtype=np.float64)
    out = np.empty_like(x)
    off = 0
    for a, d in enumerate(axes_dim):
        freqs = 1.0 / (float(theta) ** (np.arange(0, d, 2, dtype=np.float64) / d))
        ang = pos[:, a].astype(np.float64)[:, None] * freqs[None, :]          # [S, d/2]
        z = x[..., off:off + d:2] + 1j * x[..., off + 1:off + d:2]            # [S, H, d/2]
        r = z * np.exp(1j * ang)[:, None, :]
        out[..., off:off + d:2] = r.real
        out[..., off + 1:off + d:2] = r.imag
        off += d
    return out


# Flux2PosEmbed.py: 4 axes x 2 dims, positions <= 8 (test_zero / test_4d_axes).
pos_a = np.array([[0, 0, 0, 0], [1, 2, 3, 4], [5, 6, 7, 8]], dtype=np.int32)
xa = rng.randn(3, 4, 8).astype(np.float32)
fx["rope_toy_x"], fx["rope_toy_pos"] = xa, pos_a
fx["rope_toy_y"] = rope_diffusers(xa, pos_a, [2, 2, 2, 2], 10000)
# Flux2 layout: 4 x 32 dims, text ids [0,0,0,l] then image ids [0,y,x,0].
txt = np.array([[0, 0, 0, l] for l in range(8)], dtype=np.int32)
img = np.array([[0, y, x, 0] for y in range(4) for x in range(4)], dtype=np.int32)
pos_b = np.concatenate([txt, img])
xb = rng.randn(pos_b.shape[0], 3, 128).astype(np.float32)
fx["rope_flux_x"], fx["rope_flux_pos"] = xb, pos_b
fx["rope_flux_y"] = rope_diffusers(xb, pos_b, [32] * 4, 2000)
# Large positions (text l up to 511) for the drift bound of the fp32 angle recurrence.
pos_c = np.array([[0, 0, 0, l] for l in (0, 1, 17, 255, 400, 511)], dtype=np.int32)
xc = rng.randn(pos_c.shape[0], 2, 128).astype(np.float32)
fx["rope_far_x"], fx["rope_far_pos"] = xc, pos_c
fx["rope_far_y"] = rope_diffusers(xc, pos_c, [32] * 4, 10000)

# Number formats: fp32 -> bf16 (torch, round-to-nearest-even) incl. ties.
vals = np.concatenate([rng.randn(2000).astype(np.float32) * 10,
                       np.array([1.0, -1.0, 0.0, 3.0e38, 1e-40, -2.5e-39], dtype=np.float32),
                       (np.arange(64, dtype=np.uint32) * 0x8000 + 0x3F800000).view(np.float32)])
fx["bf16_in"] = vals
fx["bf16_bits"] = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)

np.savez_compressed(os.path.join(HERE, "chain_golden.npz"), **fx)
print("wrote quant_kat.json and chain_golden.npz")
