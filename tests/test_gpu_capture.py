"""The fused chain captured into a HIP graph (through torch.cuda.CUDAGraph,
launches still go through the C ABI) must reproduce the eager results on
every replay, with the program's own eager work and synchronisations in
between.  None of the library's kernels records a memset, so replays are
expected to be bit-identical to the eager launches."""
import numpy as np
import pytest
import torch

import dit_hip
from test_gpu_fused import dev_tensor, flux_positions

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager(orc, dev):
    S, D, H, I = 320, 3072, 24, 9216
    pos = torch.from_numpy(flux_positions(64, 16)).cuda()
    x = dev_tensor(orc.randn(1, (S, D)), torch.bfloat16)
    sh = dev_tensor(orc.randn(2, (D,), std=0.1), torch.float32)
    sc = dev_tensor(orc.randn(3, (D,), std=0.1), torch.float32)
    q = dev_tensor(orc.randn(4, (S, H, 128)), torch.bfloat16)
    k = dev_tensor(orc.randn(5, (S, H, 128)), torch.bfloat16)
    w = dev_tensor(orc.randn(6, (128,), mean=1.0, std=0.02), torch.float32)
    gu = dev_tensor(orc.randn(7, (S, 2 * I)), torch.bfloat16)
    gate = dev_tensor(orc.randn(8, (D,), std=0.1), torch.float32)
    gn_x = dev_tensor(orc.randn(9, (1, 64, 32, 32)), torch.bfloat16)
    tab = dit_hip.rope_table(64, 32, 10000.0)
    outs = [torch.empty((S, D), dtype=torch.bfloat16, device="cuda"),
            torch.empty((S, H, 128), dtype=torch.bfloat16, device="cuda"),
            torch.empty((S, H, 128), dtype=torch.bfloat16, device="cuda"),
            torch.empty((S, I), dtype=torch.bfloat16, device="cuda"),
            torch.empty((S, D), dtype=torch.bfloat16, device="cuda"),
            torch.empty((1, 64, 32, 32), dtype=torch.bfloat16, device="cuda")]
    ws = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")

    def chain():
        dit_hip.adaln_mod(x, sh, sc, 1e-6, out=outs[0])
        dit_hip.qk_rmsnorm_rope(q, k, w, w, pos, 32, 10000.0, 1e-6, table=tab, q_out=outs[1],
                                k_out=outs[2])
        dit_hip.swiglu(gu[:, :I], gu[:, I:], out=outs[3])
        dit_hip.gated_residual(x, outs[0], gate, out=outs[4])
        dit_hip.groupnorm_silu(gn_x, 32, None, None, 1e-6, out=outs[5], workspace=ws)

    chain()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        chain()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        chain()
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))                      # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager)):
            assert torch.equal(o.view(torch.int16), e.view(torch.int16)), f"replay {rep} output {i}"


def test_dt_graph_capture_replays_match_eager(orc, dev):
    """dt_graph_capture records one dt_graph_compute of a single-stream
    block's chain (fused adaLN, q/k QK-RMSNorm+RoPE with the SwiGLU, gated
    residual); each replay, after eager torch work has overwritten the
    outputs, reproduces the eager results bit for bit."""
    import ctypes

    import dit_hip as dh
    from graphkit import Backend
    from test_gpu_graph_ops import build_single_block_chain
    lib = dh.load()
    be = Backend()
    g, _, _, outs, _ = build_single_block_chain(orc, torch.bfloat16, 48, 3072, 24, 9216)
    for o in outs.values():
        o.d.flags |= dh.FLAG_OUTPUT
    arr, n = g._array(), len(g.nodes)
    dh.check(lib.dt_graph_compute(be.h, arr, n), "dt_graph_compute")
    dh.check(lib.dt_backend_synchronize(be.h), "sync")
    eager = {k: o.torch().clone() for k, o in outs.items()}
    ex = ctypes.c_void_p()
    dh.check(lib.dt_graph_capture(be.h, arr, n, ctypes.byref(ex)), "dt_graph_capture")
    try:
        for rep in range(3):
            for o in outs.values():
                o.torch().fill_(float("nan"))
            torch.cuda.synchronize()
            dh.check(lib.dt_graph_exec_launch(be.h, ex), "dt_graph_exec_launch")
            dh.check(lib.dt_backend_synchronize(be.h), "sync")
            for k, o in outs.items():
                assert torch.equal(o.torch().view(torch.int16), eager[k].view(torch.int16)), f"replay {rep} {k}"
    finally:
        lib.dt_graph_exec_free(ex)
        be.close()


def test_mul_mat_graphs_capture_and_replay(orc, dev):
    """Two MUL_MAT graphs of different shapes on one backend: each is
    computed eagerly, then captured, and every replay (after its output was
    overwritten) reproduces the eager product bit for bit; the eager product
    agrees with the fp32 product at the bf16 bar."""
    import ctypes

    import dit_hip as dh
    from graphkit import Backend, Graph
    lib = dh.load()

    def mm_graph(m, n, k, seed):
        g = Graph()
        w = g.leaf(dev_tensor(orc.randn(seed, (n, k), std=0.02), torch.bfloat16))
        x = g.leaf(dev_tensor(orc.randn(seed + 1, (m, k)), torch.bfloat16))
        y = g.mul_mat(w, x)
        y.d.flags |= dh.FLAG_OUTPUT
        return g, w, x, y

    be = Backend()
    try:
        for g, w, x, y in (mm_graph(40, 96, 64, 31), mm_graph(72, 160, 128, 41)):
            g.compute(be.h)
            dh.check(lib.dt_backend_synchronize(be.h), "sync")
            eager = y.torch().clone()
            ref = x.torch().float() @ w.torch().float().t()
            err = ((eager.float() - ref).norm() / ref.norm()).item()
            assert err < 1e-2, err
            ex = ctypes.c_void_p()
            dh.check(lib.dt_graph_capture(be.h, g._array(), len(g.nodes), ctypes.byref(ex)), "dt_graph_capture")
            try:
                for rep in range(3):
                    y.torch().fill_(float("nan"))
                    torch.cuda.synchronize()
                    dh.check(lib.dt_graph_exec_launch(be.h, ex), "dt_graph_exec_launch")
                    dh.check(lib.dt_backend_synchronize(be.h), "sync")
                    assert torch.equal(y.torch().view(torch.int16), eager.view(torch.int16)), f"replay {rep}"
            finally:
                lib.dt_graph_exec_free(ex)
    finally:
        be.close()
