"""Test-side graph builder: emits dt_tensor nodes the way the reference's
Runtime calls emit ggml nodes (src/ggml/Runtime.hpp), with every node's
data allocated up front as a torch tensor (gallocr's role in the
reference), then runs them through dt_graph_compute.

Shapes are given in ggml order (ne[0] fastest) to keep the node structure
one-to-one with the reference's graphs."""
import ctypes
import struct

import torch

import dit_hip as dh

_TORCH = {dh.F32: torch.float32, dh.BF16: torch.bfloat16, dh.F16: torch.float16, dh.I32: torch.int32}
_ES = {dh.F32: 4, dh.BF16: 2, dh.F16: 2, dh.I32: 4}


def fbits(v: float) -> int:
    return struct.unpack("<i", struct.pack("<f", v))[0]


class Node:
    def __init__(self, d: dh.DtTensor, data=None):
        self.d = d
        self.data = data          # torch tensor owning the memory (None for views)

    @property
    def ne(self):
        return list(self.d.ne)

    def torch(self):
        """Contiguous node data as a torch tensor of PyTorch shape."""
        return self.data


class Graph:
    def __init__(self, device="cuda"):
        self.nodes = []
        self.keep = []
        self.device = device

    # ---- tensors ----------------------------------------------------------
    def leaf(self, t: torch.Tensor) -> Node:
        t = t.contiguous() if t.dim() <= 4 else t
        self.keep.append(t)
        return Node(dh.desc(t), t)

    def _new(self, op, ne, type_, srcs, params=()):
        ne = list(ne) + [1] * (4 - len(ne))
        shape = [n for n in reversed(ne)]
        data = torch.empty(shape, dtype=_TORCH[type_], device=self.device)
        d = dh.desc(data, op)
        for i, s in enumerate(srcs):
            d.src[i] = ctypes.pointer(s.d) if s is not None else None
        for i, p in enumerate(params):
            d.op_params[i] = p
        n = Node(d, data)
        self.nodes.append(n)
        return n

    def view(self, src: Node, ne, nb, offset_bytes=0) -> Node:
        d = dh.DtTensor()
        d.type = src.d.type
        d.op = dh.OP_VIEW
        ne = list(ne) + [1] * (4 - len(ne))
        for i in range(4):
            d.ne[i] = ne[i]
        nb = list(nb)
        while len(nb) < 4:
            nb.append(nb[-1] * ne[len(nb) - 1])
        for i in range(4):
            d.nb[i] = nb[i]
        d.data = src.d.data + offset_bytes
        d.op_params[0] = ctypes.c_int32(offset_bytes & 0xFFFFFFFF).value
        d.op_params[1] = offset_bytes >> 32
        d.src[0] = ctypes.pointer(src.d)
        n = Node(d)
        self.nodes.append(n)
        return n

    def reshape(self, src: Node, ne) -> Node:
        es = _ES[src.d.type]
        ne = list(ne) + [1] * (4 - len(ne))
        nb = [es]
        for i in range(1, 4):
            nb.append(nb[-1] * ne[i - 1])
        return self.view(src, ne, nb, 0)

    # ---- ops (Runtime method names) ----------------------------------------
    def _binary(self, op, a, b):
        return self._new(op, a.ne, a.d.type, [a, b])

    def add(self, a, b):
        return self._binary(dh.OP_ADD, a, b)

    def sub(self, a, b):
        return self._binary(dh.OP_SUB, a, b)

    def mul(self, a, b):
        return self._binary(dh.OP_MUL, a, b)

    def div(self, a, b):
        return self._binary(dh.OP_DIV, a, b)

    def scale(self, a, s):
        return self._new(dh.OP_SCALE, a.ne, a.d.type, [a], [fbits(s)])

    def sigmoid(self, a):
        return self._new(dh.OP_SIGMOID, a.ne, a.d.type, [a])

    def fill(self, ne, type_, value):
        return self._new(dh.OP_FILL, ne, type_, [], [fbits(value)])

    def norm(self, a, eps):
        return self._new(dh.OP_NORM, a.ne, a.d.type, [a], [fbits(eps)])

    def rms_norm(self, a, eps):
        return self._new(dh.OP_RMS_NORM, a.ne, a.d.type, [a], [fbits(eps)])

    def rope_ext(self, a, pos, n_dims, mode, freq_base, freq_scale=1.0, ext_factor=0.0,
                 attn_factor=1.0):
        return self._new(dh.OP_ROPE, a.ne, a.d.type, [a, pos],
                         [n_dims, mode, fbits(freq_base), fbits(freq_scale), fbits(ext_factor),
                          fbits(attn_factor)])

    def concat(self, a, b, dim):
        ne = a.ne
        ne[dim] += b.ne[dim]
        return self._new(dh.OP_CONCAT, ne, a.d.type, [a, b], [dim])

    def cont(self, a, type_=None):
        return self._new(dh.OP_CPY, a.ne, type_ if type_ is not None else a.d.type, [a])

    def conv_2d_direct(self, w, x, s0=1, s1=1, p0=1, p1=1, d0=1, d1=1):
        """ggml_conv_2d_direct: w ne {K, K, Ci, Co}, x ne {W, H, Ci, N}."""
        K = w.ne[0]
        ow = (x.ne[0] + 2 * p0 - d0 * (K - 1) - 1) // s0 + 1
        oh = (x.ne[1] + 2 * p1 - d1 * (K - 1) - 1) // s1 + 1
        return self._new(dh.OP_CONV_2D_DIRECT, [ow, oh, w.ne[3], x.ne[3]], x.d.type, [w, x], [s0, s1, p0, p1, d0, d1])

    def mul_mat(self, w, x, type_=None):
        """ggml_mul_mat(w, x): out[.., m, n] = sum_k x[.., m, k] * w[n, k]
        (Runtime::mul_mat, src/ggml/Runtime.hpp:136-139), output rows of w.ne[1]."""
        ne = [w.ne[1], x.ne[1], x.ne[2], x.ne[3]]
        return self._new(dh.OP_MUL_MAT, ne, type_ if type_ is not None else x.d.type, [w, x])

    def flash_attn_ext(self, q, k, v, scale):
        """q ne {D, Sq, H, B}, k / v ne {D, Skv, H, B} -> ne {D, H, Sq, B}."""
        ne = q.ne
        return self._new(dh.OP_FLASH_ATTN_EXT, [ne[0], ne[2], ne[1], ne[3]], dh.BF16, [q, k, v], [fbits(scale)])

    def permute_tokens_heads(self, x):
        """View of x ne {D, A, B, C} as ne {D, B, A, C} (axes 1 and 2 swapped)."""
        ne, nb = x.ne, list(x.d.nb)
        return self.view(x, [ne[0], ne[2], ne[1], ne[3]], [nb[0], nb[2], nb[1], nb[3]], 0)

    def upscale(self, a, factor):
        ne = a.ne
        return self._new(dh.OP_UPSCALE, [ne[0] * factor, ne[1] * factor, ne[2], ne[3]], a.d.type, [a], [factor])

    # ---- execution ---------------------------------------------------------
    def _array(self):
        return (ctypes.POINTER(dh.DtTensor) * len(self.nodes))(*[ctypes.pointer(n.d) for n in self.nodes])

    def plan(self, outputs=()):
        """Per-node fused-into indices from dt_graph_plan (-1: runs alone)."""
        for o in outputs:
            o.d.flags |= dh.FLAG_OUTPUT
        roots = (ctypes.c_int32 * len(self.nodes))()
        dh.check(dh.load().dt_graph_plan(self._array(), len(self.nodes), roots), "dt_graph_plan")
        return list(roots)

    def plan_checked(self, outputs=()):
        """dt_graph_plan_checked on the nodes' current data pointers:
        (per-node fused-into indices, runs_at, launches held back)."""
        for o in outputs:
            o.d.flags |= dh.FLAG_OUTPUT
        n = len(self.nodes)
        roots = (ctypes.c_int32 * n)()
        runs = (ctypes.c_int32 * n)()
        held = ctypes.c_int32()
        dh.check(dh.load().dt_graph_plan_checked(self._array(), n, roots, runs, ctypes.byref(held)),
                 "dt_graph_plan_checked")
        return list(roots), list(runs), held.value

    def compute(self, backend, outputs=(), flags=0):
        """dt_graph_compute_ex: (kernels launched, nodes fused); the launches
        the address replay held back are in self.last_held."""
        for o in outputs:
            o.d.flags |= dh.FLAG_OUTPUT
        dh.check(dh.load().dt_graph_compute_ex(backend, self._array(), len(self.nodes), flags), "dt_graph_compute")
        k = ctypes.c_int32()
        f = ctypes.c_int32()
        h = ctypes.c_int32()
        dh.load().dt_graph_last_stats_ex(ctypes.byref(k), ctypes.byref(f), ctypes.byref(h))
        self.last_held = h.value
        return k.value, f.value


class Backend:
    def __init__(self):
        self.h = ctypes.c_void_p()
        dh.check(dh.load().dt_backend_init(0, ctypes.byref(self.h)), "dt_backend_init")
        dh.check(dh.load().dt_backend_set_stream(self.h, dh.stream()), "dt_backend_set_stream")

    def close(self):
        if self.h:
            dh.load().dt_backend_free(self.h)
            self.h = ctypes.c_void_p()
