"""dt_groupnorm_silu_noalloc: GroupNorm(32) + SiLU whose statistics live in
the library's own device array instead of a caller workspace (for callers
that cannot allocate).  Called through the C ABI and checked bit for bit
against dt_groupnorm_silu on the same inputs, twice in a row with the second
map smaller (the array keeps the first call's contents), in fp32 and bf16;
a map whose statistics exceed the array is refused before any device work."""
import ctypes

import numpy as np
import pytest
import torch

import dit_hip

pytestmark = pytest.mark.gpu


def _inputs(shape, dtype, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = torch.randn(shape, device="cuda", generator=g).to(dtype)
    w = torch.randn(shape[1], device="cuda", generator=g) * 0.02 + 1
    b = torch.randn(shape[1], device="cuda", generator=g) * 0.02
    return x, w, b


def _call_noalloc(x, w, b, y):
    lib = dit_hip.load()
    N, C, H, W = x.shape
    rc = lib.dt_groupnorm_silu_noalloc(ctypes.c_void_p(x.data_ptr()), N, C, H * W, 32,
                                       ctypes.c_void_p(w.data_ptr()), ctypes.c_void_p(b.data_ptr()), 1e-6, 1,
                                       ctypes.c_void_p(y.data_ptr()), dit_hip.io_type(x), dit_hip.stream())
    assert rc == 0, lib.dt_last_error().decode()


def _bits(t):
    return t.view(torch.int32 if t.element_size() == 4 else torch.int16).cpu().numpy()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_noalloc_matches_the_workspace_entry_point(dtype):
    dit_hip.load()
    for i, shape in enumerate([(1, 512, 256, 256), (1, 128, 64, 64)]):
        print(f"noalloc GroupNorm {shape} {dtype} (call {i + 1})", flush=True)
        x, w, b = _inputs(shape, dtype, 11 + i)
        want = dit_hip.groupnorm_silu(x, 32, w, b, 1e-6)
        y = torch.full_like(x, float("nan"))
        _call_noalloc(x, w, b, y)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(y), _bits(want)), f"{shape} {dtype}: differs from dt_groupnorm_silu"


def test_noalloc_refuses_maps_beyond_its_scratch():
    lib = dit_hip.load()
    x = torch.empty(1, dtype=torch.float32, device="cuda")
    # 8 x 256 channels of 1024 x 1024 fp32: 256 groups x 2049 chunks of statistics, beyond 2 MiB
    rc = lib.dt_groupnorm_silu_noalloc(ctypes.c_void_p(x.data_ptr()), 8, 256, 1024 * 1024, 32, None, None, 1e-6, 1,
                                       ctypes.c_void_p(x.data_ptr()), dit_hip.F32, dit_hip.stream())
    assert rc != 0 and b"beyond its" in lib.dt_last_error()
