"""numpy-facing wrapper of the oracle (liboracle.so, a C restatement of the
ggml CPU arithmetic the diffusers-cpp Flux2 modules emit).

Test infrastructure only: the tests, the smoke check and the CPU-baseline
leg of the benchmark may use it, as the checker (or as the timed CPU
baseline).  The product library never imports it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import POINTER, c_float, c_int, c_int32, c_int64, c_uint16, c_uint64, c_void_p

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

_lib = None


def build():
    subprocess.check_call(["make", "-s", "-C", _HERE])


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    lib = ctypes.CDLL(LIB_PATH)
    P = c_void_p
    sigs = {
        "or_mt64_nth": (c_uint64, [c_uint64, c_uint64]),
        "or_randn_f32": (None, [c_uint64, c_int64, c_float, c_float, P]),
        "or_rand_int32": (None, [c_uint64, c_int64, c_int32, c_int32, P]),
        "or_splitmix64": (c_uint64, [c_uint64]),
        "or_fnv1a64": (c_uint64, [ctypes.c_char_p]),
        "or_hash_key": (c_uint64, [c_uint64, ctypes.c_char_p]),
        "or_hash_q8_0": (None, [c_uint64, ctypes.c_char_p, c_int64, c_int64, P, c_int]),
        "or_hash_norm_weight": (None, [c_uint64, ctypes.c_char_p, c_int64, P]),
        "or_f16_to_f32": (c_float, [c_uint16]),
        "or_f32_to_f16": (c_uint16, [c_float]),
        "or_bf16_to_f32": (c_float, [c_uint16]),
        "or_f32_to_bf16": (c_uint16, [c_float]),
        "or_f32_to_bf16_n": (None, [P, c_int64, P]),
        "or_bf16_to_f32_n": (None, [P, c_int64, P]),
        "or_round_bf16_n": (None, [P, c_int64, P]),
        "or_norm_f32": (None, [P, c_int64, c_int64, c_float, P, c_int]),
        "or_rms_norm_f32": (None, [P, c_int64, c_int64, c_float, P, c_int]),
        "or_sigmoid_f32": (None, [P, c_int64, P]),
        "or_scale_f32": (None, [P, c_int64, c_float, P]),
        "or_binary_f32": (None, [c_int, P, P, P, P, P, P, P]),
        "or_concat_f32": (None, [P, P, P, P, c_int, P]),
        "or_rope_cache": (None, [c_float, c_int, c_int64, c_float, c_float, c_float, P]),
        "or_rope_normal_f32": (None, [P, P, P, P, c_int, c_float, c_float, c_float, P]),
        "or_adaln_f32": (None, [P, c_int64, c_int64, P, P, c_float, P, c_int]),
        "or_qk_rmsnorm_rope_f32": (None, [P, c_int64, c_int64, c_int64, P, c_float, P, c_int64,
                                          c_int, c_int, c_float, P, c_int]),
        "or_swiglu_f32": (None, [P, c_int64, P, c_int64, c_int64, c_int64, P, c_int]),
        "or_gated_residual_f32": (None, [P, P, P, c_int64, c_int64, P, c_int]),
        "or_groupnorm_silu_f32": (None, [P, c_int64, c_int64, c_int64, c_int64, P, P, c_float,
                                         c_int, P, c_int]),
        "or_euler_f32": (None, [P, P, c_float, c_int64, P]),
        "or_quantize_q8_0": (None, [P, c_int64, P]),
        "or_dequant_q8_0_f32": (None, [P, c_int64, P, c_int]),
        "or_quantize_q4_K": (None, [P, c_int64, P]),
        "or_dequant_q4_K_f32": (None, [P, c_int64, P, c_int]),
        "or_q4_K_scale_min": (None, [c_int, P, P, P]),
        "or_conv2d_f32": (None, [P, c_int64, c_int64, c_int64, c_int64, P, c_int64, c_int64, c_int64, P,
                                 c_int, P, c_int]),
        "or_linear_f32": (None, [P, c_int64, c_int64, c_int64, P, c_int64, c_int64, P, P, c_int64,
                                 c_int]),
        "or_linear_q8_0_ggml": (None, [P, c_int64, c_int64, c_int64, P, c_int64, P, P, c_int64, c_int]),
        "or_attention_f32": (None, [P, P, P, P, c_int64, c_int64, c_int64, c_int64, P, P, P, P,
                                    c_float, c_int]),
        "or_max_threads": (c_int, []),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return c_void_p(a.ctypes.data)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- generator / formats ---------------------------------------------------

def mt64_nth(seed: int, n: int) -> int:
    return int(load().or_mt64_nth(seed, n))


def randn(seed: int, shape, mean=0.0, std=1.0) -> np.ndarray:
    out = np.empty(int(np.prod(shape)), dtype=np.float32)
    load().or_randn_f32(seed, out.size, mean, std, _p(out))
    return out.reshape(shape)


def randint(seed: int, shape, lo: int, hi: int) -> np.ndarray:
    out = np.empty(int(np.prod(shape)), dtype=np.int32)
    load().or_rand_int32(seed, out.size, lo, hi, _p(out))
    return out.reshape(shape)


def hash_key(seed: int, path: str) -> int:
    return int(load().or_hash_key(seed, path.encode()))


def hash_q8_0(seed: int, path: str, rows: int, cols: int, threads=0) -> np.ndarray:
    """Q8_0 block bytes of a hash-drawn [rows, cols] Linear weight (the rule
    dit_cli --hash-weights applies; stated in oracle.c)."""
    assert cols % 32 == 0
    out = np.empty(rows * cols // 32 * 34, dtype=np.uint8)
    load().or_hash_q8_0(seed, path.encode(), rows, cols, _p(out), threads)
    return out


def hash_norm_weight(seed: int, path: str, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    load().or_hash_norm_weight(seed, path.encode(), n, _p(out))
    return out


def tensor_seed(index: int) -> int:
    """Seed of the index-th generated tensor of a workload."""
    return 0x5EED0000 + index


def to_bf16_bits(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, dtype=np.uint16)
    load().or_f32_to_bf16_n(_p(x), x.size, _p(out))
    return out


def from_bf16_bits(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    out = np.empty(b.shape, dtype=np.float32)
    load().or_bf16_to_f32_n(_p(b), b.size, _p(out))
    return out


def round_bf16(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    load().or_round_bf16_n(_p(x), x.size, _p(out))
    return out


def f16_to_f32(h: int) -> float:
    return float(load().or_f16_to_f32(h))


def f32_to_f16(f: float) -> int:
    return int(load().or_f32_to_f16(f))


# ---- single ops ------------------------------------------------------------

def norm(x, eps, threads=0):
    x = _f32(x)
    y = np.empty_like(x)
    load().or_norm_f32(_p(x), x.size // x.shape[-1], x.shape[-1], eps, _p(y), threads)
    return y


def rms_norm(x, eps, threads=0):
    x = _f32(x)
    y = np.empty_like(x)
    load().or_rms_norm_f32(_p(x), x.size // x.shape[-1], x.shape[-1], eps, _p(y), threads)
    return y


def sigmoid(x):
    x = _f32(x)
    y = np.empty_like(x)
    load().or_sigmoid_f32(_p(x), x.size, _p(y))
    return y


def _ggml_ne_nb(a: np.ndarray):
    """ggml ne/nb (int64[4]) of an ndarray of <= 4 dims (strides honoured)."""
    ne = list(a.shape)[::-1] + [1] * (4 - a.ndim)
    nb = [s for s in a.strides[::-1]]
    while len(nb) < 4:
        nb.append(nb[-1] * ne[len(nb) - 1] if nb else a.itemsize)
    return np.array(ne, dtype=np.int64), np.array(nb, dtype=np.int64)


def binary(op: int, a, b):
    """ggml binary op (0 add, 1 sub, 2 mul, 3 div): b repeats into a's shape."""
    a = np.asarray(a, dtype=np.float32)
    b = np.asarray(b, dtype=np.float32)
    nea, nba = _ggml_ne_nb(a)
    neb, nbb = _ggml_ne_nb(b)
    out = np.empty(a.shape, dtype=np.float32)
    load().or_binary_f32(op, c_void_p(a.ctypes.data), _p(nea), _p(nba), c_void_p(b.ctypes.data),
                         _p(neb), _p(nbb), _p(out))
    return out


def concat(a, b, dim_ggml: int):
    a, b = _f32(a), _f32(b)
    nea, _ = _ggml_ne_nb(a)
    neb, _ = _ggml_ne_nb(b)
    axis = a.ndim - 1 - dim_ggml
    out = np.empty(np.concatenate([a, b], axis=axis).shape, dtype=np.float32)
    load().or_concat_f32(_p(a), _p(nea), _p(b), _p(neb), dim_ggml, _p(out))
    return out


def rope_cache(p: float, n_dims: int, ne0: int, freq_base: float, freq_scale=1.0, attn_factor=1.0):
    out = np.empty(ne0, dtype=np.float32)
    load().or_rope_cache(p, n_dims, ne0, freq_base, freq_scale, attn_factor, _p(out))
    return out


def rope_normal(x, pos, n_dims, freq_base, freq_scale=1.0, attn_factor=1.0):
    """x: ndarray [B, S, H, D] (any strides, PyTorch order); pos: int32 [S]."""
    x = np.asarray(x, dtype=np.float32)
    while x.ndim < 4:
        x = x[None]
    ne, nb = _ggml_ne_nb(x)
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    out = np.empty(x.shape, dtype=np.float32)
    load().or_rope_normal_f32(c_void_p(x.ctypes.data), _p(ne), _p(nb), _p(pos), n_dims, freq_base,
                              freq_scale, attn_factor, _p(out))
    return out


# ---- chains ----------------------------------------------------------------

def adaln(x, shift, scale, eps=1e-6, threads=0):
    x = _f32(x)
    y = np.empty_like(x)
    cols = x.shape[-1]
    load().or_adaln_f32(_p(x), x.size // cols, cols, _p(_f32(shift)), _p(_f32(scale)), eps, _p(y),
                        threads)
    return y


def qk_rmsnorm_rope(x, w, pos, axis_dim, freq_base, eps=1e-6, threads=0):
    """x: [tokens, heads, head_dim]; pos: int32 [tokens, n_axes]."""
    x = _f32(x)
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    tokens, heads, head_dim = x.shape
    y = np.empty_like(x)
    load().or_qk_rmsnorm_rope_f32(_p(x), tokens, heads, head_dim, _p(_f32(w)), eps, _p(pos),
                                  pos.shape[1], pos.shape[1], axis_dim, freq_base, _p(y), threads)
    return y


def swiglu(g, u, threads=0):
    g, u = _f32(g), _f32(u)
    cols = g.shape[-1]
    y = np.empty_like(g)
    load().or_swiglu_f32(_p(g), cols, _p(u), cols, g.size // cols, cols, _p(y), threads)
    return y


def gated_residual(h, o, gate, threads=0):
    h, o = _f32(h), _f32(o)
    cols = h.shape[-1]
    y = np.empty_like(h)
    load().or_gated_residual_f32(_p(h), _p(o), _p(_f32(gate)), h.size // cols, cols, _p(y), threads)
    return y


def groupnorm_silu(x, groups, w=None, b=None, eps=1e-6, silu=True, threads=0, out=None):
    x = _f32(x)
    N, C = x.shape[0], x.shape[1]
    HW = x.size // (N * C)
    y = np.empty_like(x) if out is None else out
    assert y.shape == x.shape and y.dtype == np.float32 and y.flags["C_CONTIGUOUS"]
    wp = _p(_f32(w)) if w is not None else None
    bp = _p(_f32(b)) if b is not None else None
    load().or_groupnorm_silu_f32(_p(x), N, C, HW, groups, wp, bp, eps, 1 if silu else 0, _p(y),
                                 threads)
    return y


def euler(x, v, dt):
    x, v = _f32(x), _f32(v)
    y = np.empty_like(x)
    load().or_euler_f32(_p(x), _p(v), dt, x.size, _p(y))
    return y


# ---- matmul and attention ------------------------------------------------------

def conv2d(x, w, b=None, padding=None, up2=False, threads=0):
    """x: [N, Ci, H, W]; w: [Co, Ci, K, K]; b: [Co] or None -> [N, Co, OH, OW]
    (stride 1; padding (K-1)/2 by default; up2: on the nearest 2x upscale)."""
    x, w = _f32(x), _f32(w)
    N, Ci, H, W = x.shape
    Co, Ci2, K, K2 = w.shape
    assert Ci2 == Ci and K2 == K
    P = (K - 1) // 2 if padding is None else padding
    Hs, Ws = (2 * H, 2 * W) if up2 else (H, W)
    y = np.empty((N, Co, Hs + 2 * P - K + 1, Ws + 2 * P - K + 1), dtype=np.float32)
    bp = _p(_f32(b)) if b is not None else None
    load().or_conv2d_f32(_p(x), N, Ci, H, W, _p(w), Co, K, P, bp, 1 if up2 else 0, _p(y), threads)
    return y


class Q8_0Weight:
    """A [rows, cols] Linear weight held as ggml Q8_0 blocks (rows of cols/32
    blocks of 34 bytes).  linear() multiplies by it with ggml's CPU Q8_0
    arithmetic (activations quantised to Q8_0, or_linear_q8_0_ggml), as the
    reference's mul_mat does for a Q8_0 weight."""

    def __init__(self, blocks, rows: int, cols: int):
        assert cols % 32 == 0
        self.blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        assert self.blocks.size == rows * cols // 32 * 34
        self.shape = (rows, cols)

    def dequantize(self, threads=0) -> np.ndarray:
        return dequantize(self.blocks, self.shape[0] * self.shape[1], 8, threads).reshape(self.shape)


def linear(x, w, b=None, threads=0):
    """x: [..., K]; w: [N, K] (PyTorch Linear weight) or a Q8_0Weight; b: [N]
    or None -> [..., N].  An fp32 weight: fp32 products, exact-order sum
    rounded once; a Q8_0Weight: ggml's Q8_0 x Q8_0 arithmetic."""
    if isinstance(w, Q8_0Weight):
        x = _f32(x)
        N, K = w.shape
        assert x.shape[-1] == K
        M = x.size // K
        y = np.empty(x.shape[:-1] + (N,), dtype=np.float32)
        bp = _p(_f32(b)) if b is not None else None
        load().or_linear_q8_0_ggml(_p(x), M, K, K, _p(w.blocks), N, bp, _p(y), N, threads)
        return y
    x, w = _f32(x), _f32(w)
    K = x.shape[-1]
    N = w.shape[0]
    assert w.shape[1] == K
    M = x.size // K
    y = np.empty(x.shape[:-1] + (N,), dtype=np.float32)
    bp = _p(_f32(b)) if b is not None else None
    load().or_linear_f32(_p(x), M, K, K, _p(w), N, K, bp, _p(y), N, threads)
    return y


def attention(q, k, v, scale=None, threads=0):
    """q: [seq_q, heads, head_dim]; k, v: [seq_kv, heads, head_dim] -> [seq_q, heads, head_dim]."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    sq, heads, hd = q.shape
    skv = k.shape[0]
    scale = 1.0 / np.sqrt(hd) if scale is None else scale
    o = np.empty_like(q)
    st = lambda t: (c_int64 * 2)(t.shape[1] * t.shape[2], t.shape[2])
    load().or_attention_f32(_p(q), _p(k), _p(v), _p(o), heads, sq, skv, hd, st(q), st(k), st(v),
                            st(o), float(scale), threads)
    return o


# ---- quantisation ------------------------------------------------------------

def quantize(x, qtype: int) -> np.ndarray:
    """Row-major float32 matrix -> ggml block bytes (qtype 8 = Q8_0, 12 = Q4_K)."""
    x = _f32(x)
    qk, bs = (32, 34) if qtype == 8 else (256, 144)
    assert x.shape[-1] % qk == 0
    out = np.empty(x.size // qk * bs, dtype=np.uint8)
    fn = load().or_quantize_q8_0 if qtype == 8 else load().or_quantize_q4_K
    fn(_p(x), x.size, _p(out))
    return out


def dequantize(b, n: int, qtype: int, threads=0, out=None) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32) if out is None else out
    assert out.size == n and out.dtype == np.float32 and out.flags["C_CONTIGUOUS"]
    fn = load().or_dequant_q8_0_f32 if qtype == 8 else load().or_dequant_q4_K_f32
    fn(_p(b), n, _p(out), threads)
    return out


def q4_K_scale_min(j: int, scales12) -> tuple[int, int]:
    s = np.ascontiguousarray(scales12, dtype=np.uint8)
    sc = np.zeros(1, dtype=np.uint8)
    m = np.zeros(1, dtype=np.uint8)
    load().or_q4_K_scale_min(j, _p(s), _p(sc), _p(m))
    return int(sc[0]), int(m[0])


def max_threads() -> int:
    return int(load().or_max_threads())
