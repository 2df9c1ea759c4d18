"""CPU-side checks of the C ABI: the library loads, exports every function
include/dit_hip.h declares, its descriptor layout matches the C compiler's,
argument validation rejects bad calls before touching a device, and the
host-side helpers (RoPE table, workspace sizing, invariant division) are
right.  No kernel is launched here."""
import ctypes
import os
import re
import subprocess
import tempfile

import numpy as np
import pytest

import dit_hip
from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "dit_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dt_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = dit_hip.load()
    names = declared_functions()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"
    # and the Python binding declares a signature for each of them
    assert sorted(dit_hip.exported_symbols()) == names


def test_descriptor_layout_matches_c():
    src = r"""
    #include <stddef.h>
    #include <stdio.h>
    #include "dit_hip.h"
    int main(void) {
        printf("%zu %zu %zu %zu %zu %zu %zu %zu %zu\n", sizeof(dt_tensor),
               offsetof(dt_tensor, type), offsetof(dt_tensor, op), offsetof(dt_tensor, ne),
               offsetof(dt_tensor, nb), offsetof(dt_tensor, data), offsetof(dt_tensor, op_params),
               offsetof(dt_tensor, src), offsetof(dt_tensor, flags));
        return 0;
    }
    """
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "l.c")
        open(c, "w").write(src)
        exe = os.path.join(d, "l")
        subprocess.check_call(["gcc", "-I", os.path.dirname(HEADER), c, "-o", exe])
        got = [int(v) for v in subprocess.check_output([exe]).split()]
    T = dit_hip.DtTensor
    want = [ctypes.sizeof(T), T.type.offset, T.op.offset, T.ne.offset, T.nb.offset, T.data.offset,
            T.op_params.offset, T.src.offset, T.flags.offset]
    assert got == want


def test_type_ids_match_ggml():
    text = open(HEADER).read()
    for name, val in (("F32", 0), ("F16", 1), ("Q8_0", 8), ("Q4_K", 12), ("I32", 26), ("BF16", 30)):
        assert re.search(rf"DT_TYPE_{name}\s*=\s*{val}\b", text)
        assert getattr(dit_hip, name) == val


def _err(rc):
    assert rc != 0
    return dit_hip.load().dt_last_error().decode()


def test_validation_rejects_before_launch():
    lib = dit_hip.load()
    P = ctypes.c_void_p
    dummy = P(16)
    # unsupported io type
    msg = _err(lib.dt_adaln_mod(dummy, 4, 64, 64, dummy, dummy, dummy, 64, 1e-6, 99, None))
    assert "io_type" in msg
    # stride smaller than cols
    assert "stride" in _err(lib.dt_adaln_mod(dummy, 4, 64, 32, dummy, dummy, dummy, 64, 1e-6, 30, None))
    # head_dim != n_axes * axis_dim
    msg = _err(lib.dt_qk_rmsnorm_rope(dummy, None, dummy, None, 4, 2, 128, 256, 128, 256, 128,
                                      dummy, None, 1e-6, dummy, 4, 4, 16, 1e4, None, 0, 30, None))
    assert "head_dim" in msg
    # Q4_K needs cols % 256 == 0; Q8_0 row_bytes too small
    assert "multiple" in _err(lib.dt_dequant(dummy, 12, 2, 100, 1000, dummy, 100, 30, None))
    assert "row_bytes" in _err(lib.dt_dequant(dummy, 8, 2, 64, 10, dummy, 64, 30, None))
    # unsupported quant type / dst type
    assert "qtype" in _err(lib.dt_dequant(dummy, 2, 2, 64, 68, dummy, 64, 30, None))
    assert "dst_type" in _err(lib.dt_dequant(dummy, 8, 2, 64, 68, dummy, 64, 1, None))
    # group norm: groups must divide C, workspace must be big enough
    assert "bad shape" in _err(lib.dt_groupnorm_silu(dummy, 1, 30, 16, 32, None, None, 1e-6, 1, dummy,
                                                     dummy, 1 << 20, 30, None))
    assert "workspace" in _err(lib.dt_groupnorm_silu(dummy, 1, 64, 16, 32, None, None, 1e-6, 1, dummy,
                                                     dummy, 8, 30, None))
    # rope_ext: only NORMAL mode
    d = dit_hip.DtTensor()
    d.type, d.data = dit_hip.F32, 16
    for i in range(4):
        d.ne[i], d.nb[i] = (8 if i == 0 else 1), (4 if i == 0 else 32)
    assert "mode" in _err(lib.dt_op_rope_ext(ctypes.byref(d), dummy, ctypes.byref(d), 8, 2, 1e4, 1.0,
                                             0.0, 1.0, None))
    # binary: src1 must broadcast into src0
    e = dit_hip.DtTensor()
    e.type, e.data = dit_hip.F32, 16
    for i in range(4):
        e.ne[i], e.nb[i] = (3 if i == 0 else 1), (4 if i == 0 else 12)
    assert "broadcast" in _err(lib.dt_op_binary(0, ctypes.byref(d), ctypes.byref(e), ctypes.byref(d), None))
    # zero rows is a no-op success
    assert lib.dt_adaln_mod(None, 0, 64, 64, None, None, None, 64, 1e-6, 30, None) == 0


def test_rope_table_matches_oracle_cache(orc):
    tab = dit_hip.rope_table(512, 32, 10000.0, device="cpu").numpy()
    for p in (0, 1, 2, 63, 64, 300, 511):
        want = orc.rope_cache(float(p), 32, 32, 10000.0)
        assert np.array_equal(tab[p], want), p
    tab2 = dit_hip.rope_table(8, 2, 2000.0, device="cpu").numpy()
    for p in range(8):
        assert np.array_equal(tab2[p], orc.rope_cache(float(p), 2, 2, 2000.0))


def test_groupnorm_workspace_bytes():
    lib = dit_hip.load()
    # one (K, sum, sumsq per chunk) record per (n, g), chunks of 1024 elements (the scalar path's)
    assert lib.dt_groupnorm_workspace_bytes(1, 128, 1024 * 1024, 32) == 32 * (2 * 4096 + 1) * 8
    assert lib.dt_groupnorm_workspace_bytes(2, 4, 9, 2) == 2 * 2 * (2 * 1 + 1) * 8
    assert lib.dt_groupnorm_workspace_bytes(1, 30, 16, 32) == 0


def test_fastdiv_arithmetic():
    # The kernels' row index: q = (umulhi(n, m) + n) >> s with host-made (m, s).
    def make(d):
        s = 0
        while (1 << s) < d:
            s += 1
        return ((((1 << 32) * ((1 << s) - d)) // d) + 1) & 0xFFFFFFFF, s

    rng = np.random.RandomState(0)
    for d in list(range(1, 3000)) + [int(v) for v in rng.randint(1, 1 << 30, 500)]:
        m, s = make(d)
        ns = [0, 1, d - 1, d, d + 1, (1 << 31) - 1] + [int(v) for v in rng.randint(0, 1 << 31, 50)]
        for n in ns:
            assert (((n * m) >> 32) + n) >> s == n // d


def test_conv2d_packed_weight_type():
    """DT_TYPE_CONV2D_PACKED (101): a conv weight {K, K, Ci, Co} packed once
    at load, dt_conv2d_packed_bytes long (Co to 128, Ci to 32, bf16); the
    descriptor calls size it by that count (a copy past it is refused before
    any device call)."""
    lib = dit_hip.load()
    text = open(HEADER).read()
    assert "DT_TYPE_CONV2D_PACKED = 101" in text
    assert lib.dt_conv2d_packed_bytes(512, 512, 3) == 512 * 9 * 512 * 2      # 4.7 MB, no padding
    assert lib.dt_conv2d_packed_bytes(3, 3, 3) == 128 * 9 * 32 * 2
    assert lib.dt_conv2d_packed_bytes(4, 4, 2) == 0                          # K in {1, 3} only
    t = dit_hip.DtTensor()
    t.type = 101
    for i, n in enumerate((3, 3, 512, 512)):
        t.ne[i] = n
    t.data = 0x10000  # never dereferenced: the size check fails first
    buf = ctypes.create_string_buffer(16)
    total = 512 * 9 * 512 * 2
    assert lib.dt_tensor_set(ctypes.byref(t), buf, total, 1, None) != 0
    assert "exceed the tensor's %d bytes" % total in lib.dt_last_error().decode()
    t.ne[1] = 1  # not a square kernel: not a packed weight
    assert lib.dt_tensor_set(ctypes.byref(t), buf, 0, 1, None) != 0
    assert "not supported" in lib.dt_last_error().decode()


@pytest.mark.parametrize("type_,ne", [
    (0, (1 << 31, 1 << 31, 1 << 31, 1)),      # F32: element count past 2^63
    (30, (1 << 62, 4, 1, 1)),                 # BF16: bytes past 2^63
    (8, (1 << 62, 1 << 10, 1, 1)),            # Q8_0 blocks x rows past 2^63
    (100, (1 << 31, 1 << 31, 1, 1)),          # Q8_0_SPLIT: N K past 2^60
    (0, (4, -1, 1, 1)),                       # a negative size
])
def test_tensor_copies_refuse_overflowing_descriptors(type_, ne):
    """dt_tensor_set / dt_tensor_get bound a copy by the tensor's byte extent;
    a descriptor whose extent overflows 64 bits (or has a negative size) is
    refused before any device call, not wrapped into a small or negative
    bound."""
    lib = dit_hip.load()
    t = dit_hip.DtTensor()
    t.type = type_
    for i, v in enumerate(ne):
        t.ne[i] = v
    es = {0: 4, 30: 2}.get(type_, 1)
    t.nb[0] = es
    for i in range(1, 4):
        t.nb[i] = t.nb[i - 1] * max(ne[i - 1], 1) if type_ in (0, 30) else 0
    t.data = 0x10000  # never dereferenced
    buf = ctypes.create_string_buffer(16)
    for fn in (lib.dt_tensor_set, lib.dt_tensor_get):
        assert fn(ctypes.byref(t), buf, 0, 16, None) != 0
        msg = lib.dt_last_error().decode()
        assert "not supported" in msg or "not contiguous" in msg, msg


def test_zero_sized_calls_are_no_ops_without_a_device():
    """Every entry point of the chain, the dequantisation and GroupNorm takes
    an empty input (zero rows, tokens or images) as a successful no-op: it
    launches nothing, so in this container (no GPU) any HIP call it made
    would fail.  The data pointers are dummies that must not be touched."""
    lib = dit_hip.load()
    P = ctypes.c_void_p(0x10000)           # 64 KiB-aligned, never dereferenced
    BF16, Q8, Q4 = dit_hip.BF16, dit_hip.Q8_0, dit_hip.Q4_K
    D, I = 3072, 9216
    calls = {
        "dt_adaln_mod": (P, 0, D, D, P, P, P, D, 1e-6, BF16, None),
        "dt_gated_residual_adaln": (P, D, P, D, P, P, D, P, P, P, D, 0, D, 1e-6, BF16, None),
        "dt_gated_residual": (P, D, P, D, P, P, D, 0, D, BF16, None),
        "dt_swiglu": (P, 2 * I, P, 2 * I, P, I, 0, I, BF16, None),
        "dt_euler_step": (P, P, 0.1, P, 0, BF16, None),
        "dt_qk_rmsnorm_rope": (P, P, P, P, 0, 24, 128, D, 128, D, 128, P, P, 1e-6, P, 4, 4, 32, 1e4,
                               None, 0, BF16, None),
        "dt_qk_rmsnorm_rope_swiglu": (P, P, P, P, 0, 24, 128, D, 128, D, 128, P, P, 1e-6, P, 4, 4, 32, 1e4,
                                      None, 0, P, 2 * I, P, 2 * I, P, I, 0, I, BF16, None),
        # empty outputs may come as null pointers (an empty torch tensor has none)
        "dt_qk_rmsnorm_rope null outputs": (P, P, None, None, 0, 24, 128, D, 128, D, 128, P, P, 1e-6, P, 4, 4,
                                            32, 1e4, None, 0, BF16, None),
        "dt_groupnorm_silu": (P, 0, 512, 128 * 128, 32, P, P, 1e-6, 1, P, P,
                              lib.dt_groupnorm_workspace_bytes(0, 512, 128 * 128, 32), BF16, None),
        "dt_groupnorm_silu_noalloc": (P, 0, 512, 128 * 128, 32, P, P, 1e-6, 1, P, BF16, None),
    }
    for qt, bs in ((Q8, 34), (Q4, 144)):
        calls[f"dt_dequant q{qt}"] = (P, qt, 0, D, D // (32 if qt == Q8 else 256) * bs, P, D, BF16, None)
    failed = {}
    for name, args in calls.items():
        rc = getattr(lib, name.split()[0])(*args)
        if rc != 0:
            failed[name] = lib.dt_last_error().decode()
    assert not failed, failed


def test_prepare_repeats_the_recorded_call():
    """dit_hip.prepare runs a wrapper once and returns a launch that repeats
    the same C-ABI call with the converted arguments (here the host-side
    RoPE table fill, so no device is needed)."""
    import torch
    table, launch = dit_hip.prepare(dit_hip.rope_table, 16, 32, 10000.0, device="cpu")
    want = table.clone()
    table.zero_()
    assert launch() == 0                       # the same pointer, filled again
    assert torch.equal(table, want)
    assert dit_hip.load() is not None and not isinstance(dit_hip.load(), dit_hip._Recorder)


def test_q8_0_split_layout_sizes():
    """DT_TYPE_Q8_0_SPLIT: codes [N][K] then fp32 scales [K/32][N] at the
    codes rounded up to 256 bytes."""
    lib = dit_hip.load()
    assert lib.dt_q8_0_split_scale_offset(3072, 3072) == 3072 * 3072
    assert lib.dt_q8_0_split_scale_offset(33, 64) == 2304          # 2112 -> 2304
    assert lib.dt_q8_0_split_bytes(33, 64) == 2304 + 2 * 33 * 4
    assert lib.dt_q8_0_split_bytes(9216, 3072) == 9216 * 3072 + 96 * 9216 * 4
