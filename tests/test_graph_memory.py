"""The executor's memory-hazard replay on the CPU (dt_graph_plan_checked on
host descriptors; no kernel runs).

ggml_gallocr (the reference's allocator, src/ggml/Context.hpp:118-135)
frees a node's memory after its last reader in node order and hands it to
later nodes.  A fused launch that reads an input later than node order (a
chain reads its first node's inputs at its last node; residual + adaLN reads
o at the next block's norm) would then read another node's data.  Each case
places the nodes' data the way such an allocator could, and checks that the
plan keeps the launch in node order (or unfused) exactly when it must."""
import torch

import dit_hip as dh
from graphkit import Graph

C, R = 256, 4


def _bf16(g, *shape):
    return g.leaf(torch.zeros(shape, dtype=torch.bfloat16))


def _f32(g, *shape):
    return g.leaf(torch.zeros(shape, dtype=torch.float32))


def _adaln_graph(clobber=False, inplace=False, partial=False):
    """x = a + b; y = LN(x) * (1 + scale) + shift, with an unrelated node z
    between the norm and the modulation in node order."""
    g = Graph(device="cpu")
    a, b, c, d = (_bf16(g, R, C) for _ in range(4))
    scale, shift = _f32(g, C), _f32(g, C)
    x = g.add(a, b)
    n = g.norm(x, 1e-6)
    z = g.add(c, d)
    s1 = g.add(scale, g.fill([C], dh.F32, 1.0))
    m = g.mul(n, s1)
    y = g.add(m, shift)
    if clobber:      # x is dead after the norm in node order: z may take its memory
        z.d.data = x.d.data
    if inplace:      # the whole chain in place over x (norm, mul, add are in-place ops)
        y.d.data = x.d.data
    if partial:
        y.d.data = x.d.data + 128
    return g, x, n, z, y


def _i(g, node):
    return next(i for i, t in enumerate(g.nodes) if t is node)


def test_adaln_fuses_when_memory_is_distinct():
    g, x, n, z, y = _adaln_graph()
    roots, runs, held = g.plan_checked(outputs=[y, z])
    assert roots[_i(g, n)] == _i(g, y) and held == 0


def test_adaln_kept_unfused_when_its_input_is_reused():
    g, x, n, z, y = _adaln_graph(clobber=True)
    roots, runs, held = g.plan_checked(outputs=[y, z])
    assert roots[_i(g, n)] == -1 and held == 1
    # the plan without the replay (dt_graph_plan) still fuses: the replay made the difference
    assert g.plan(outputs=[y, z])[_i(g, n)] == _i(g, y)


def test_adaln_in_place_over_its_input_stays_fused():
    g, x, n, z, y = _adaln_graph(inplace=True)
    roots, runs, held = g.plan_checked(outputs=[y, z])
    assert roots[_i(g, n)] == _i(g, y) and held == 0


def test_partial_overlap_of_output_and_input_is_not_fused():
    g, x, n, z, y = _adaln_graph(partial=True)
    roots, runs, held = g.plan_checked(outputs=[y, z])
    assert roots[_i(g, n)] == -1 and held == 1


def _res_adaln_graph(clobber=False):
    """r = h + gate * o (stored: read again after the next adaLN), then
    y = LN(r) * (1 + scale) + shift; the (1 + scale) ADD runs between them."""
    g = Graph(device="cpu")
    h, o1, o2 = (_bf16(g, R, C) for _ in range(3))
    gate, scale, shift = _f32(g, C), _f32(g, C), _f32(g, C)
    o = g.add(o1, o2)
    go = g.mul(o, gate)
    r = g.add(h, go)
    n = g.norm(r, 1e-6)
    s1 = g.add(scale, g.fill([C], dh.F32, 1.0))
    m = g.mul(n, s1)
    y = g.add(m, shift)
    r2 = g.add(r, y)
    if clobber:      # o is dead after gate * o in node order: the (1 + scale) vector may take it
        s1.d.data = o.d.data
    return g, o, r, n, y, r2


def test_residual_moves_into_the_next_adaln_when_memory_allows():
    g, o, r, n, y, r2 = _res_adaln_graph()
    roots, runs, held = g.plan_checked(outputs=[r2])
    assert runs[_i(g, r)] == _i(g, y) and held == 0


def test_residual_stays_in_place_when_its_input_is_reused():
    """The residual runs at its own position (gated residual kernel) and the
    adaLN stays fused: only the move is undone."""
    g, o, r, n, y, r2 = _res_adaln_graph(clobber=True)
    roots, runs, held = g.plan_checked(outputs=[r2])
    assert held == 1
    assert runs[_i(g, r)] == _i(g, r)
    assert roots[_i(g, n)] == _i(g, y)


def test_compute_flags_are_checked():
    lib = dh.load()
    rc = lib.dt_graph_compute_ex(None, None, 0, 0)
    assert rc != 0 and b"null backend" in lib.dt_last_error()
