"""The streaming probe bench.py sets the chain beside
(diffusers-cpp_amd/probe/stream_probe.hip) does the work it is timed for:
every vector of every stream is read and written, in both segments."""
import ctypes
import os

import pytest
import torch

from conftest import PKG

pytestmark = pytest.mark.gpu


def _probe():
    lib = ctypes.CDLL(os.path.join(PKG, "lib", "libdit_probe.so"))
    fn = lib.dt_stream_probe
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_void_p),
                   ctypes.POINTER(ctypes.c_int64), ctypes.c_void_p]
    return fn


def test_stream_probe_touches_every_vector(dev):
    fn = _probe()
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    n0, n1 = 1000 * 512 + 37, 3 * 512 + 5          # 16-byte vectors; partial last workgroups
    r = lambda n: torch.randint(0, 2 ** 31 - 1, (n, 4), generator=g, device="cuda", dtype=torch.int32)
    a0, b0, a1, b1 = r(n0), r(n0), r(n1), r(n1)
    y0, z0, y1 = (torch.full_like(t, -1) for t in (a0, a0, a1))
    ins = (ctypes.c_void_p * 4)(a0.data_ptr(), b0.data_ptr(), a1.data_ptr(), b1.data_ptr())
    outs = (ctypes.c_void_p * 4)(y0.data_ptr(), z0.data_ptr(), y1.data_ptr(), None)
    assert fn(ins, outs, (ctypes.c_int64 * 2)(n0, n1), None) == 0
    torch.cuda.synchronize()
    assert torch.equal(y0, a0 ^ b0) and torch.equal(z0, a0 + b0) and torch.equal(y1, a1 ^ b1)


def test_stream_probe_rejects_misaligned(dev):
    fn = _probe()
    a = torch.zeros(64, dtype=torch.int32, device="cuda")
    ins = (ctypes.c_void_p * 4)(a.data_ptr() + 4, None, None, None)
    outs = (ctypes.c_void_p * 4)(a.data_ptr(), None, None, None)
    assert fn(ins, outs, (ctypes.c_int64 * 2)(4, 0), None) == 1
