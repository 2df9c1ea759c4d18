"""Pins for the oracle's Flux2 compositions (oracle/flux2.py) on the CPU.

Each test is a property the mathematics fixes, built so that a plausible
composition mistake fails it (wrong modulation chunk, wrong stream paired
with the position rows, scale and shift swapped in norm_out, a missing
timestep scaling, sin/cos halves swapped).  Where a test's power is not
obvious, a planted mistake in the oracle (patched in the test, on the CPU)
is shown to fail the same check.

Reference modules restated by the functions pinned here:
  timestep_proj  src/diffusers/models/embeddings/Timesteps.cpp:17-45
  single_block   src/diffusers/models/transformers/flux2/Flux2SingleTransformerBlock.hpp:36-72
  double_block   src/diffusers/models/transformers/flux2/Flux2TransformerBlock.hpp:45-117
  model          src/diffusers/models/transformers/flux2/Flux2Transformer2DModel.cpp:111-231,
                 src/diffusers/models/normalization/AdaLayerNormContinuous.inl:26-43
"""
import math

import numpy as np
import pytest

from conftest import assert_fp32

D, HEADS, AXIS = 64, 2, 8          # head_dim 32 = 4 axes x 8 dims
MLP = 3 * D
THETA, EPS = 2000.0, 1e-6
N_TXT, GRID = 5, 3                 # 5 text tokens, a 3x3 image grid (9 tokens)
N_IMG = GRID * GRID


@pytest.fixture(scope="module")
def fx(orc):
    import oracle.flux2 as f2
    return f2


def _pos():
    txt = [[0, 0, 0, l] for l in range(N_TXT)]
    img = [[0, y, x, 0] for y in range(GRID) for x in range(GRID)]
    return np.array(txt, np.int32), np.array(img, np.int32)


def _params(orc, shapes, seed, std=0.1):
    P = {}
    for i, (name, shape) in enumerate(sorted(shapes.items())):
        mean = 1.0 if name.endswith(("norm_q.weight", "norm_k.weight", "norm_added_q.weight",
                                     "norm_added_k.weight")) else 0.0
        P[name] = orc.randn(seed + i, shape, mean=mean, std=0.05 if mean else std)
    return P


def _layernorm64(x, eps=EPS):
    x = np.asarray(x, np.float64)
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)
    return (x - m) / np.sqrt(v + eps)


def _silu64(x):
    x = np.asarray(x, np.float64)
    return x / (1.0 + np.exp(-x))


# ---- timestep_proj -------------------------------------------------------------

def test_timestep_proj_at_zero_is_cos_then_sin(fx):
    tp = fx.timestep_proj(0.0)
    assert tp.shape == (1, 256)
    assert np.array_equal(tp[0, :128], np.ones(128, np.float32))
    assert np.array_equal(tp[0, 128:], np.zeros(128, np.float32))
    # flip_sin_to_cos=False puts sin first (Timesteps.cpp:34-37)
    tp2 = fx.timestep_proj(0.0, flip_sin_to_cos=False)
    assert np.array_equal(tp2[0, :128], np.zeros(128, np.float32))


def test_timestep_proj_first_frequency_is_one(fx):
    t = 0.7312
    tp = fx.timestep_proj(t)[0].astype(np.float64)
    assert abs(tp[0] - math.cos(t)) <= 1e-6
    assert abs(tp[128] - math.sin(t)) <= 1e-6
    # both halves take the same argument per index
    assert np.max(np.abs(tp[:128] ** 2 + tp[128:] ** 2 - 1.0)) <= 1e-6


def test_timestep_proj_frequency_ladder(fx):
    """sin(t f_i) / t -> f_i for small t: f_i = 10000^(-i/128), the exponent
    divided by half_dim - shift = 128 (a divisor of 127 would give 1e-4 for
    the last index instead of 1.0746e-4)."""
    t = 1e-3
    tp = fx.timestep_proj(t)[0].astype(np.float64)
    f = tp[128:] / t
    want = 10000.0 ** (-np.arange(128) / 128.0)
    assert np.max(np.abs(f / want - 1.0)) <= 2e-5
    assert abs(f[127] - 1.0746e-4) / 1.0746e-4 < 1e-3


# ---- single_block ----------------------------------------------------------------

def _single_setup(orc, fx, seed=0x5EED1000):
    P = _params(orc, fx.single_block_param_shapes(D, HEADS), seed)
    txt, img = _pos()
    pos = np.concatenate([txt, img])
    x = orc.randn(seed + 100, (N_TXT + N_IMG, D))
    return P, pos, x


def _mod(orc, seed, n_sets, zero=()):
    """Modulation vector of n_sets (shift, scale, gate) triples; chunks listed
    in `zero` are zeroed."""
    m = orc.randn(seed, (3 * n_sets * D,), std=0.5)
    for c in zero:
        m[c * D:(c + 1) * D] = 0.0
    return m


def test_single_block_zero_gate_returns_input(orc, fx):
    P, pos, x = _single_setup(orc, fx)
    mod = _mod(orc, 7, 1, zero=(2,))           # shift, scale non-zero; gate (chunk 2) zero
    y = fx.single_block(x, mod, pos, P, HEADS, THETA, AXIS, EPS)
    assert np.array_equal(y, x)


def test_single_block_zero_output_projection_returns_input(orc, fx):
    P, pos, x = _single_setup(orc, fx)
    P["attn.to_out.attn.weight"][:] = 0.0
    P["attn.to_out.mlp.weight"][:] = 0.0
    y = fx.single_block(x, _mod(orc, 8, 1), pos, P, HEADS, THETA, AXIS, EPS)
    assert np.array_equal(y, x)


def _uniform_attention_case(orc, fx):
    """q = k = 0 makes attention the token average of v; v = n (identity
    weight), to_out.attn = identity, the MLP branch zeroed.  Then every row
    of the block output is x + gate * ((1 + scale) * mean_s LN(x_s) + shift)."""
    P, pos, x = _single_setup(orc, fx)
    eye = np.eye(D, dtype=np.float32)
    P["attn.to_qkv_mlp_proj.q.weight"][:] = 0.0
    P["attn.to_qkv_mlp_proj.k.weight"][:] = 0.0
    P["attn.to_qkv_mlp_proj.v.weight"][:] = eye
    P["attn.to_out.attn.weight"][:] = eye
    P["attn.to_out.mlp.weight"][:] = 0.0
    mod = _mod(orc, 9, 1)
    shift, scale, gate = (mod[i * D:(i + 1) * D].astype(np.float64) for i in range(3))
    mean_n = _layernorm64(x).mean(0)
    want = x.astype(np.float64) + gate * ((1.0 + scale) * mean_n + shift)
    return P, pos, x, mod, want


def test_single_block_modulation_chunk_order(orc, fx):
    """Chunks 0, 1, 2 of the modulation are shift, scale, gate
    (Flux2Modulation.hpp:24-41)."""
    P, pos, x, mod, want = _uniform_attention_case(orc, fx)
    y = fx.single_block(x, mod, pos, P, HEADS, THETA, AXIS, EPS)
    assert_fp32(y, want, what="single_block chunk order")


def test_single_block_chunk_order_check_catches_a_swap(orc, fx, monkeypatch):
    """A planted mistake (scale and shift swapped in the split) fails the
    check above."""
    P, pos, x, mod, want = _uniform_attention_case(orc, fx)
    real = fx._split_mod
    monkeypatch.setattr(fx, "_split_mod", lambda m, s: [[c[1], c[0], c[2]] for c in real(m, s)])
    y = fx.single_block(x, mod, pos, P, HEADS, THETA, AXIS, EPS)
    with pytest.raises(AssertionError):
        assert_fp32(y, want, what="planted swap")


# ---- double_block ----------------------------------------------------------------

def _tied_double(orc, fx, seed=0x5EED2000):
    """A double block whose txt and img streams share every weight with one
    single block, and whose feed-forwards are zeroed: the double block is
    then the single block's attention over the joint txt|img sequence."""
    Ps, pos, x = _single_setup(orc, fx, seed)
    Ps["attn.to_out.mlp.weight"][:] = 0.0
    Pd = _params(orc, fx.double_block_param_shapes(D, HEADS), seed + 500)
    a = "attn."
    for img, txt, src in (("to_q", "add_q_proj", "q"), ("to_k", "add_k_proj", "k"), ("to_v", "add_v_proj", "v")):
        Pd[a + img + ".weight"] = Ps[a + "to_qkv_mlp_proj." + src + ".weight"].copy()
        Pd[a + txt + ".weight"] = Ps[a + "to_qkv_mlp_proj." + src + ".weight"].copy()
    for img, txt, src in (("norm_q", "norm_added_q", "norm_q"), ("norm_k", "norm_added_k", "norm_k")):
        Pd[a + img + ".weight"] = Ps[a + src + ".weight"].copy()
        Pd[a + txt + ".weight"] = Ps[a + src + ".weight"].copy()
    Pd[a + "to_out.0.weight"] = Ps[a + "to_out.attn.weight"].copy()
    Pd[a + "to_add_out.weight"] = Ps[a + "to_out.attn.weight"].copy()
    Pd["ff.linear_out.weight"][:] = 0.0
    Pd["ff_context.linear_out.weight"][:] = 0.0
    mod1 = _mod(orc, 11, 1)
    mod2 = np.concatenate([mod1, _mod(orc, 12, 1)])   # first triple shared; second set only feeds the FF
    return Ps, Pd, pos, x, mod1, mod2


def test_double_block_reduces_to_single_block_on_joint_sequence(orc, fx):
    """The joint sequence is txt first, and each stream is rotated by its own
    position rows (Flux2TransformerBlock.hpp:45-117 with Flux2Attention's
    txt|img concat): with tied weights the double block's two outputs are the
    single block's rows [:n_txt] and [n_txt:]."""
    Ps, Pd, pos, x, mod1, mod2 = _tied_double(orc, fx)
    e, h = x[:N_TXT], x[N_TXT:]
    e2, h2 = fx.double_block(h, e, mod2, mod2, pos, Pd, HEADS, THETA, AXIS, EPS)
    y = fx.single_block(x, mod1, pos, Ps, HEADS, THETA, AXIS, EPS)
    assert_fp32(e2, y[:N_TXT], what="txt rows")
    assert_fp32(h2, y[N_TXT:], what="img rows")


def test_double_block_position_pairing_is_observable(orc, fx):
    """The reduction above is sensitive to which rows of `pos` each stream
    takes: handing the positions over in img|txt order breaks it."""
    Ps, Pd, pos, x, mod1, mod2 = _tied_double(orc, fx)
    e, h = x[:N_TXT], x[N_TXT:]
    swapped = np.concatenate([pos[N_TXT:], pos[:N_TXT]])
    e2, h2 = fx.double_block(h, e, mod2, mod2, swapped[:N_TXT + N_IMG], Pd, HEADS, THETA, AXIS, EPS)
    y = fx.single_block(x, mod1, pos, Ps, HEADS, THETA, AXIS, EPS)
    with pytest.raises(AssertionError):
        assert_fp32(np.concatenate([e2, h2]), y, what="planted position swap")


def test_double_block_zero_gates_return_inputs(orc, fx):
    Pd = _params(orc, fx.double_block_param_shapes(D, HEADS), 0x5EED3000)
    txt, img = _pos()
    pos = np.concatenate([txt, img])
    h = orc.randn(1, (N_IMG, D))
    e = orc.randn(2, (N_TXT, D))
    zero_gates = (2, 5)                     # gate_msa, gate_mlp of each stream
    mi, mt = _mod(orc, 3, 2, zero_gates), _mod(orc, 4, 2, zero_gates)
    e2, h2 = fx.double_block(h, e, mi, mt, pos, Pd, HEADS, THETA, AXIS, EPS)
    assert np.array_equal(h2, h) and np.array_equal(e2, e)


def _ff_collapse_case(orc, fx, stream):
    """Attention outputs zeroed and the stream's scale_mlp (chunk 4) = -1:
    the FF input (1 + scale_mlp) * LN(h) + shift_mlp collapses to shift_mlp,
    so the stream's output is h + gate_mlp * W_out (g sigma(g) u) with
    g = W_gate shift_mlp, u = W_up shift_mlp (chunks 3, 4, 5 = shift, scale,
    gate of the second set; Flux2TransformerBlock.hpp:89-111)."""
    Pd = _params(orc, fx.double_block_param_shapes(D, HEADS), 0x5EED4000)
    Pd["attn.to_out.0.weight"][:] = 0.0
    Pd["attn.to_add_out.weight"][:] = 0.0
    txt, img = _pos()
    pos = np.concatenate([txt, img])
    h = orc.randn(5, (N_IMG, D))
    e = orc.randn(6, (N_TXT, D))
    mi, mt = _mod(orc, 7, 2), _mod(orc, 8, 2)
    m = mi if stream == "img" else mt
    m[4 * D:5 * D] = -1.0
    ff = "ff." if stream == "img" else "ff_context."
    sh, gt = m[3 * D:4 * D].astype(np.float64), m[5 * D:6 * D].astype(np.float64)
    g = Pd[ff + "linear_in_gate.weight"].astype(np.float64) @ sh
    u = Pd[ff + "linear_in_up.weight"].astype(np.float64) @ sh
    row = Pd[ff + "linear_out.weight"].astype(np.float64) @ (g / (1.0 + np.exp(-g)) * u)
    base = h if stream == "img" else e
    want = base.astype(np.float64) + gt * row
    return Pd, pos, h, e, mi, mt, want


@pytest.mark.parametrize("stream", ["img", "txt"])
def test_double_block_feed_forward_chunk_order(orc, fx, stream):
    Pd, pos, h, e, mi, mt, want = _ff_collapse_case(orc, fx, stream)
    e2, h2 = fx.double_block(h, e, mi, mt, pos, Pd, HEADS, THETA, AXIS, EPS)
    assert_fp32(h2 if stream == "img" else e2, want, what=f"{stream} FF")


def test_double_block_ff_check_catches_swapped_mod_sets(orc, fx):
    """A planted mistake (the two modulation sets exchanged) fails it."""
    Pd, pos, h, e, mi, mt, want = _ff_collapse_case(orc, fx, "img")
    mi_swapped = np.concatenate([mi[3 * D:], mi[:3 * D]])
    e2, h2 = fx.double_block(h, e, mi_swapped, mt, pos, Pd, HEADS, THETA, AXIS, EPS)
    with pytest.raises(AssertionError):
        assert_fp32(h2, want, what="planted set swap")


# ---- model ------------------------------------------------------------------------

def _model_cfg(n_double=0, n_single=0):
    return {"num_attention_heads": HEADS, "attention_head_dim": D // HEADS, "in_channels": D,
            "joint_attention_dim": 24, "num_layers": n_double, "num_single_layers": n_single,
            "axes_dims_rope": [AXIS] * 4, "rope_theta": THETA, "eps": EPS}


def _model_inputs(orc):
    txt, img = _pos()
    hidden = orc.randn(21, (N_IMG, D))
    text = orc.randn(22, (N_TXT, 24))
    return hidden, text, img, txt


def _identity_embedders(P):
    P["x_embedder.weight"] = np.eye(D, dtype=np.float32)
    P["proj_out.weight"] = np.eye(D, dtype=np.float32)


def test_model_norm_out_scale_is_the_first_chunk(orc, fx):
    """With no blocks and identity embedders the model is
    LN(h) * (1 + scale) + shift with (scale, shift) = chunk(emb, 2)
    (AdaLayerNormContinuous.inl:30-40).  Zeroing the second half of the
    norm_out weight leaves y1 = LN(h) * (1 + e); zeroing the first half
    leaves y2 = LN(h) + e, for the same e.  So y1 - n == n * (y2 - n)."""
    cfg = _model_cfg()
    P = _params(orc, fx.model_param_shapes(cfg), 0x5EED5000, std=0.3)
    _identity_embedders(P)
    hidden, text, img, txt = _model_inputs(orc)
    W = P["norm_out.linear.weight"]
    Pa, Pb = dict(P), dict(P)
    Pa["norm_out.linear.weight"] = np.concatenate([W[:D], np.zeros_like(W[D:])])
    Pb["norm_out.linear.weight"] = np.concatenate([np.zeros_like(W[:D]), W[:D]])
    y1 = fx.model(hidden, text, 0.41, img, txt, Pa, cfg).astype(np.float64)
    y2 = fx.model(hidden, text, 0.41, img, txt, Pb, cfg).astype(np.float64)
    n = _layernorm64(hidden)
    e = y2 - n
    assert np.max(np.abs(e)) > 1e-2                       # the modulation is not trivially zero
    assert_fp32(y1, n * (1.0 + e), tol=2e-5, what="scale first")


def test_model_timestep_chain(orc, fx):
    """timestep * 1000 -> Timesteps -> linear_1 -> SiLU -> linear_2 (temb);
    norm_out's shift = W SiLU(temb).  With linear_1 rows selecting channel 0
    (cos(1000 t)), linear_2 = I and norm_out = [0; I], the output is
    LN(h) + SiLU(SiLU(cos(1000 t))) in every element."""
    cfg = _model_cfg()
    P = _params(orc, fx.model_param_shapes(cfg), 0x5EED6000)
    _identity_embedders(P)
    sel = np.zeros((D, 256), np.float32)
    sel[:, 0] = 1.0
    P["time_guidance_embed.timestep_embedder.linear_1.weight"] = sel
    P["time_guidance_embed.timestep_embedder.linear_2.weight"] = np.eye(D, dtype=np.float32)
    P["norm_out.linear.weight"] = np.concatenate([np.zeros((D, D), np.float32), np.eye(D, dtype=np.float32)])
    hidden, text, img, txt = _model_inputs(orc)
    t = 0.37
    y = fx.model(hidden, text, t, img, txt, P, cfg)
    c = _silu64(_silu64(math.cos(1000.0 * np.float64(np.float32(t)))))
    assert abs(c - _silu64(_silu64(math.cos(t)))) > 0.1     # the x1000 is observable
    assert_fp32(y, _layernorm64(hidden) + c, tol=2e-5, what="timestep chain")


def test_model_double_then_nothing_equals_single(orc, fx):
    """The model's joint layout: positions txt|img and streams cat(txt, img)
    before the single blocks, image rows sliced out after.  A model of one
    tied double block (FF zeroed) equals a model of one single block."""
    Ps, Pd, pos, x, mod1, mod2 = _tied_double(orc, fx, 0x5EED7000)
    cfg_d, cfg_s = _model_cfg(n_double=1), _model_cfg(n_single=1)
    base = _params(orc, fx.model_param_shapes(_model_cfg()), 0x5EED7800)
    _identity_embedders(base)
    Wm = orc.randn(0x5EED7900, (3 * D, D), std=0.1)
    Md = dict(base)
    Md.update({"transformer_blocks.0." + k: v for k, v in Pd.items()})
    extra = orc.randn(0x5EED7A00, (3 * D, D), std=0.1)
    Md["double_stream_modulation_img.linear.weight"] = np.concatenate([Wm, extra])
    Md["double_stream_modulation_txt.linear.weight"] = np.concatenate([Wm, extra])
    Ms = dict(base)
    Ms.update({"single_transformer_blocks.0." + k: v for k, v in Ps.items()})
    Ms["single_stream_modulation.linear.weight"] = Wm
    hidden, text, img, txt = _model_inputs(orc)
    yd = fx.model(hidden, text, 0.5, img, txt, Md, cfg_d)
    ys = fx.model(hidden, text, 0.5, img, txt, Ms, cfg_s)
    assert_fp32(yd, ys, what="double vs single model")
    # and the block did something: the output is not the no-block model's
    y0 = fx.model(hidden, text, 0.5, img, txt, base, _model_cfg())
    assert np.max(np.abs(ys - y0)) > 1e-3


def test_model_is_equivariant_to_image_token_order(orc, fx):
    """Moving image tokens together with their position rows moves the output
    rows the same way: each token is rotated by its own row of txt|img
    positions (Flux2Transformer2DModel.cpp:157-169).  Positions handed to the
    blocks in any other order break it (checked on the same inputs)."""
    cfg = _model_cfg(n_double=1, n_single=1)
    P = _params(orc, fx.model_param_shapes(cfg), 0x5EED8000, std=0.3)
    hidden, text, img, txt = _model_inputs(orc)
    perm = np.random.default_rng(3).permutation(N_IMG)
    y1 = fx.model(hidden, text, 0.5, img, txt, P, cfg)
    y2 = fx.model(hidden[perm], text, 0.5, img[perm], txt, P, cfg)
    assert_fp32(y2, y1[perm], what="equivariance")
    # positions matter: keeping the rows of img in place changes the output
    y3 = fx.model(hidden[perm], text, 0.5, img, txt, P, cfg)
    assert np.max(np.abs(y3 - y1[perm])) > 1e-4


def test_model_single_stream_modulation_takes_silu_of_temb(orc, fx):
    """One single block in the uniform-attention form, norm_out zeroed (so it
    is a plain LayerNorm) and temb = SiLU(cos(1000 t)) in every channel: the
    block's modulation is W_mod SiLU(temb) (Flux2Modulation.hpp:14-22), and
    the output is LN(x_img + gate * ((1 + scale) * mean_s LN(x_s) + shift))
    over the joint txt|img sequence."""
    cfg = _model_cfg(n_single=1)
    P = _params(orc, fx.model_param_shapes(cfg), 0x5EED9000)
    _identity_embedders(P)
    b = "single_transformer_blocks.0.attn."
    eye = np.eye(D, dtype=np.float32)
    P[b + "to_qkv_mlp_proj.q.weight"][:] = 0.0
    P[b + "to_qkv_mlp_proj.k.weight"][:] = 0.0
    P[b + "to_qkv_mlp_proj.v.weight"] = eye.copy()
    P[b + "to_out.attn.weight"] = eye.copy()
    P[b + "to_out.mlp.weight"][:] = 0.0
    sel = np.zeros((D, 256), np.float32)
    sel[:, 0] = 1.0
    P["time_guidance_embed.timestep_embedder.linear_1.weight"] = sel
    P["time_guidance_embed.timestep_embedder.linear_2.weight"] = eye.copy()
    P["norm_out.linear.weight"][:] = 0.0
    hidden, text, img, txt = _model_inputs(orc)
    t = 0.23
    y = fx.model(hidden, text, t, img, txt, P, cfg)
    c = _silu64(math.cos(1000.0 * np.float64(np.float32(t))))            # temb, every channel
    mod = P["single_stream_modulation.linear.weight"].astype(np.float64).sum(1) * _silu64(c)
    shift, scale, gate = mod[:D], mod[D:2 * D], mod[2 * D:]
    e = text.astype(np.float64) @ P["context_embedder.weight"].astype(np.float64).T
    x = np.concatenate([e, hidden.astype(np.float64)])
    m = _layernorm64(x).mean(0)
    want = _layernorm64(x[N_TXT:] + gate * ((1.0 + scale) * m + shift))
    assert_fp32(y, want, tol=2e-5, what="single-stream modulation")


def test_model_image_stream_takes_the_img_modulation(orc, fx):
    """A double block whose image-stream gates (chunks 2 and 5 of
    double_stream_modulation_img) are zero leaves the image rows alone, so the
    model equals the no-block model, while the text stream's gates are not
    zero (Flux2Transformer2DModel.cpp:140-145, 178-186)."""
    cfg = _model_cfg(n_double=1)
    P = _params(orc, fx.model_param_shapes(cfg), 0x5EEDA000, std=0.3)
    W = P["double_stream_modulation_img.linear.weight"]
    W[2 * D:3 * D] = 0.0
    W[5 * D:6 * D] = 0.0
    hidden, text, img, txt = _model_inputs(orc)
    y = fx.model(hidden, text, 0.5, img, txt, P, cfg)
    base = {k: v for k, v in P.items() if not k.startswith("transformer_blocks.")}
    y0 = fx.model(hidden, text, 0.5, img, txt, base, _model_cfg())
    assert np.array_equal(y, y0)
    Wt = P["double_stream_modulation_txt.linear.weight"]
    assert np.abs(Wt[2 * D:3 * D]).max() > 0 and np.abs(Wt[5 * D:6 * D]).max() > 0
