"""Benchmark of the fused Flux2 DiT elementwise chain on one MI355X.

Workload (one "step" = the elementwise work of one Flux2 single-stream
block between its GEMMs, over one synthetic batch, all inputs resident in
HBM, bf16 activations, fp32 math), as two fused launches in block order:
  gated residual + adaLN   r = h + gate * o (the previous block's residual,
                           stored) and y = (1 + scale) * LayerNorm(r) + shift
                           (this block's modulated norm), h, o [4608, 3072]
  QK-RMSNorm+RoPE + SwiGLU q, k [4608, 24, 128], 4 axes x 32 dims, theta 1e4,
                           positions: 512 text tokens [0,0,0,l] then a 64x64
                           image grid; gate | up = [4608, 18432] -> [4608, 9216]
Algorithmic bytes per step: every distinct input read once and every output
written once at its I/O dtype (broadcast vectors and tables counted once).

Timed steps rotate through NSETS independent buffer sets (about 1.9 GB in
all, far above the 256 MB last-level cache), so every step reads its inputs
from HBM.  Two schedules of the same step are timed: eager launches and a
HIP graph of the two launches; `value` = whole-step algorithmic GB/s of the
faster (both are reported).  Each schedule is timed after at least --warmup
untimed steps of itself and at least 0.2 s of them, so the clocks have
settled (`warmup_steps_run` reports how many ran).  The same block order
with the four standalone kernels (gated residual, adaLN of r, QK, SwiGLU)
is timed as a graph for comparison.

`stream_probe_*` is the streaming ceiling the chain is set beside: trivial
launches with the two fused launches' exact access shapes on the same
buffers (16-byte non-temporal loads and stores), timed the same ways;
`frac_of_stream_probe` = probe time / chain time (per step, and per launch
under `kernels`).  `roofline` is the dominant launch (QK+SwiGLU): its mean
duration over back-to-back launches cycling the buffer sets, HIP events
around the run on the stream it is launched on (single cold launches, which
add the dispatch latency, are reported beside it).  `cpu_baseline` is the
oracle's C restatement of the same chain (fp32, OpenMP) on a bounded
sample, timed on this host's cores; `other_workloads` holds the same for the
single-stream block (1536 x 3072, with the block's GPU time beside it), the
weight dequantisation and the GroupNorm maps.  `secondary` times the
dequantisation and GroupNorm kernels the same two ways.

`sec_per_denoise_step` is one full Flux2-klein-4B-shaped transformer step
(5 double + 20 single blocks, hidden 3072, 24x128 heads, 4096 image tokens of
128 features + 512 text tokens of width 2560, timestep 0.5) run by the C++
driver (diffusers-cpp_amd/bin/dit_cli) as a child process: Q8_0 weights
drawn N(0, 0.02) and dequantised once to bf16, bf16 activations, inputs and
weights resident in HBM, median wall time per step of the recorded graph,
replayed as one HIP graph per step (host inputs uploaded before each).
`denoise_step_q8_0_weights` is the same step with the Linear weights kept as
Q8_0 (dequantised inside the GEMMs; same outputs bit for bit);
`denoise_step_eager_launches` the bf16 step launched kernel by kernel after
the fusion pass each step.

Prints ONE JSON line.
"""
import argparse
import json
import os
import statistics
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "diffusers-cpp_amd")
sys.path.insert(0, PKG)

HBM_PEAK_GBS = 8000.0
MIN_WARM_S = 0.2  # least untimed load before each timed schedule
MFMA_PEAK_TFLOPS = 2500.0  # dense bf16
NSETS = 4
S, D, H, HD, I = 4608, 3072, 24, 128, 9216
N_TXT, GRID = 512, 64


def alg_bytes():
    """Algorithmic bytes of the two fused launches of a step and of the four
    standalone kernels they replace."""
    e = 2  # bf16
    qk = 4 * S * H * HD * e + 2 * HD * 4 + S * 4 * 4 + N_TXT * 32 * 4  # q,k in/out, w, pos, table
    sw = 3 * S * I * e                                                # gate, up in; out
    fused = {"residual_adaln": 4 * S * D * e + 3 * D * 4,              # h, o in; r, y out; 3 vectors
             "qk_swiglu": qk + sw}
    standalone = {"gated_residual": 3 * S * D * e + D * 4, "adaln": 2 * S * D * e + 2 * D * 4,
                  "qk_rmsnorm_rope": qk, "swiglu": sw}
    return fused, standalone


def positions():
    import numpy as np
    txt = [[0, 0, 0, l] for l in range(N_TXT)]
    img = [[0, y, x, 0] for y in range(GRID) for x in range(GRID)]
    return np.array(txt + img, dtype=np.int32)


def make_inputs(torch, dev, seed=0x5EED0000):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def rn(shape, std=1.0, mean=0.0, dtype=torch.bfloat16):
        t = torch.randn(shape, generator=g, device=dev, dtype=torch.float32) * std + mean
        return t.to(dtype)

    import dit_hip
    pos = torch.from_numpy(positions()).to(dev)
    return {
        "h": rn((S, D)), "o": rn((S, D)), "gate": rn((D,), 0.1, dtype=torch.float32),
        "shift": rn((D,), 0.1, dtype=torch.float32), "scale": rn((D,), 0.1, dtype=torch.float32),
        "q": rn((S, H, HD)), "k": rn((S, H, HD)),
        "wq": rn((HD,), 0.02, 1.0, torch.float32), "wk": rn((HD,), 0.02, 1.0, torch.float32),
        "pos": pos, "table": dit_hip.rope_table(N_TXT, 32, 10000.0, device=dev),
        "gu": rn((S, 2 * I)),
        "r": torch.empty((S, D), dtype=torch.bfloat16, device=dev),
        "y": torch.empty((S, D), dtype=torch.bfloat16, device=dev),
        "qo": torch.empty((S, H, HD), dtype=torch.bfloat16, device=dev),
        "ko": torch.empty((S, H, HD), dtype=torch.bfloat16, device=dev),
        "sw": torch.empty((S, I), dtype=torch.bfloat16, device=dev),
    }


def chain_kernels(t):
    """The step's two fused launches, in block order."""
    import dit_hip
    gu = t["gu"]
    return {
        "residual_adaln": lambda: dit_hip.gated_residual_adaln(
            t["h"], t["o"], t["gate"], t["shift"], t["scale"], 1e-6, r_out=t["r"], out=t["y"]),
        "qk_swiglu": lambda: dit_hip.qk_rmsnorm_rope_swiglu(
            t["q"], t["k"], t["wq"], t["wk"], t["pos"], 32, 10000.0, gu[:, :I], gu[:, I:], 1e-6,
            table=t["table"], q_out=t["qo"], k_out=t["ko"], out=t["sw"]),
    }


def standalone_kernels(t):
    """The same step as the four standalone kernels, in block order."""
    import dit_hip
    gu = t["gu"]
    return {
        "gated_residual": lambda: dit_hip.gated_residual(t["h"], t["o"], t["gate"], out=t["r"]),
        "adaln": lambda: dit_hip.adaln_mod(t["r"], t["shift"], t["scale"], 1e-6, out=t["y"]),
        "qk_rmsnorm_rope": lambda: dit_hip.qk_rmsnorm_rope(
            t["q"], t["k"], t["wq"], t["wk"], t["pos"], 32, 10000.0, 1e-6, table=t["table"],
            q_out=t["qo"], k_out=t["ko"]),
        "swiglu": lambda: dit_hip.swiglu(gu[:, :I], gu[:, I:], out=t["sw"]),
    }


class Flusher:
    """Writes 1 GiB (four times the 256 MB last-level cache) so the next
    launch reads its operands from HBM."""

    def __init__(self, torch, dev):
        self.buf = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        self.i = 0

    def __call__(self):
        self.i += 1
        self.buf.fill_(self.i & 0xFF)


def time_cold(torch, fn, n, flush, samples=False):
    """Median duration of fn() over n launches, each bracketed by its own HIP
    events on the launch stream, with the cache flushed before (outside) each
    bracket (samples=True: every duration, in seconds)."""
    st = torch.cuda.current_stream()
    fn()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(n)]
    for a, b in ev:
        flush()
        a.record(st)
        fn()
        b.record(st)
    torch.cuda.synchronize()
    ts = [a.elapsed_time(b) * 1e-3 for a, b in ev]
    return ts if samples else statistics.median(ts)


def time_stream(torch, fns, reps):
    """Per-launch time of back-to-back launches cycling over fns (one closure
    per buffer set; the sets together exceed the 256 MB last-level cache, so
    every launch reads from HBM), HIP events around the whole run on the
    launch stream: what a kernel costs inside a step, without the dispatch
    latency an event pair around a single launch adds."""
    st = torch.cuda.current_stream()
    for f in fns:
        f()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for i in range(reps):
        fns[i % len(fns)]()
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e-3 / reps


def _sets_for(set_bytes, cap=16):
    """Buffer sets whose total exceeds 1 GiB (4x the last-level cache)."""
    return int(max(2, min(cap, -(-(1 << 30) // set_bytes))))


def probe_kernels(t):
    """Trivial-math launches with the two fused launches' access shapes on
    the same buffers (diffusers-cpp_amd/probe/stream_probe.hip): h, o -> r, y;
    then q, k -> q', k' plus the two 85 MB halves of gate|up -> the SwiGLU
    output.  Each stream is read or written once with 16-byte non-temporal
    accesses, as in the kernels."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(PKG, "lib", "libdit_probe.so"))
    fn = lib.dt_stream_probe
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_void_p),
                   ctypes.POINTER(ctypes.c_int64), ctypes.c_void_p]
    gu, half = t["gu"], t["gu"].numel() // 2

    def launch(ins, outs, ns):
        a_in = (ctypes.c_void_p * 4)(*ins)
        a_out = (ctypes.c_void_p * 4)(*outs)
        a_n = (ctypes.c_int64 * 2)(*ns)

        def run():
            import torch
            rc = fn(a_in, a_out, a_n, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            if rc:
                raise RuntimeError(f"dt_stream_probe failed ({rc})")
        return run

    p = lambda x: x.data_ptr()
    v = lambda x: x.numel() * x.element_size() // 16
    return {
        "residual_adaln": launch([p(t["h"]), p(t["o"]), None, None], [p(t["r"]), p(t["y"]), None, None],
                                 [v(t["h"]), 0]),
        "qk_swiglu": launch([p(t["q"]), p(t["k"]), p(gu), p(gu) + half * gu.element_size()],
                            [p(t["qo"]), p(t["ko"]), p(t["sw"]), None], [v(t["q"]), half * gu.element_size() // 16]),
    }


def cold_torch_copy(torch, dev, flush):
    """One 256 MiB torch device copy, timed as single cold launches after a
    cache flush (dispatch latency included): a calibration figure for the
    cold-launch columns, not a streaming ceiling (the ceilings at the path's
    byte shapes come from the back-to-back ceiling sweep)."""
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    src.fill_(1)
    t = time_cold(torch, lambda: dst.copy_(src), 10, flush)
    return 2 * src.numel() / t / 1e9


DEQ_SHAPES = ((3072, 9216), (9216, 3072), (3072, 3072))      # the weight-dequantisation workload
GN_SHAPES = ((1, 512, 128, 128), (1, 512, 256, 256), (1, 256, 512, 512), (1, 128, 1024, 1024))
GN_DECODER_EXTRA = ((1, 512, 512, 512), (1, 256, 1024, 1024))   # the decoder's other GroupNorm maps


def secondary(torch, dev, flush):
    """Configs measured beside the chain: weight dequantisation (Q8_0 and
    Q4_K -> bf16 at the three matrix shapes) and GroupNorm(32)+SiLU at the
    four VAE-decoder workload shapes and the decoder's two other map sizes."""
    import dit_hip
    out = {}
    def entry(nbytes, t_stream, t_single):
        return {"us": round(t_stream * 1e6, 2), "alg_MB": round(nbytes / 1e6, 2),
                "GBs": round(nbytes / t_stream / 1e9, 1), "frac_hbm": round(nbytes / t_stream / 1e9 / HBM_PEAK_GBS, 3),
                "us_single_launch": round(t_single * 1e6, 2),
                "frac_hbm_single_launch": round(nbytes / t_single / 1e9 / HBM_PEAK_GBS, 3)}

    for rows, cols in DEQ_SHAPES:
        for tag, qt, qk, bs in (("q8_0", dit_hip.Q8_0, 32, 34), ("q4_K", dit_hip.Q4_K, 256, 144)):
            name = f"dequant_{tag}_{rows}x{cols}_bf16"
            nbytes = rows * cols // qk * bs + rows * cols * 2
            sets = []
            for _ in range(_sets_for(nbytes)):
                src = torch.randint(0, 256, (rows * cols // qk * bs,), dtype=torch.uint8, device=dev)
                view = src.view(-1, bs)
                view[:, 1] &= 0x3B                    # keep fp16 scales finite
                if qt == dit_hip.Q4_K:
                    view[:, 3] &= 0x3B
                sets.append((src, torch.empty((rows, cols), dtype=torch.bfloat16, device=dev)))
            fns = [dit_hip.prepare(dit_hip.dequant, s_, qt, rows, cols, out=y_)[1] for s_, y_ in sets]
            t = time_stream(torch, fns, 4 * len(fns))
            t1 = time_cold(torch, fns[0], 10, flush)
            out[name] = entry(nbytes, t, t1)
            del sets, fns
    for shape in GN_SHAPES + GN_DECODER_EXTRA:
        for dt, es in ((torch.float32, 4), (torch.bfloat16, 2)):
            numel = shape[0] * shape[1] * shape[2] * shape[3]
            nbytes = 2 * numel * es
            w = torch.randn(shape[1], device=dev) * 0.02 + 1
            b = torch.randn(shape[1], device=dev) * 0.02
            ws = torch.empty(dit_hip.load().dt_groupnorm_workspace_bytes(1, shape[1], shape[2] * shape[3], 32),
                             dtype=torch.uint8, device=dev)
            sets = [(torch.randn(shape, device=dev).to(dt), torch.empty(shape, dtype=dt, device=dev))
                    for _ in range(_sets_for(nbytes, 8))]
            fns = [dit_hip.prepare(dit_hip.groupnorm_silu, x_, 32, w, b, 1e-6, out=y_, workspace=ws)[1]
                   for x_, y_ in sets]
            t = time_stream(torch, fns, 4 * len(fns))
            t1 = time_cold(torch, fns[0], 6, flush)
            name = "groupnorm_silu_" + "x".join(map(str, shape)) + ("_f32" if es == 4 else "_bf16")
            out[name] = entry(nbytes, t, t1)
            del sets, fns
            torch.cuda.empty_cache()
    return out


def vae_measurements(torch, dev, flush, reps=6):
    """The VAE decoder's 3x3 convs (dt_conv2d with a workspace: channel-last
    copy + DMA-fed MFMA kernel; bias) and their GroupNorm(32)+SiLU at the
    decoder's shapes: GroupNorm two-pass (statistics + apply) against the
    statistics from the conv epilogue (dt_conv2d_gn) + one apply pass."""
    import dit_hip
    out = {}
    for shape, co in (((1, 512, 128, 128), 512), ((1, 512, 256, 256), 512), ((1, 256, 512, 512), 256),
                      ((1, 128, 1024, 1024), 128)):
        for dt, tag, es in ((torch.bfloat16, "bf16", 2), (torch.float32, "f32", 4)):
            x = torch.randn(shape, device=dev).to(dt)
            wp = dit_hip.conv2d_pack(torch.randn(co, shape[1], 3, 3, device=dev) * 0.02)
            b = torch.randn(co, device=dev) * 0.1
            gw = torch.randn(co, device=dev) * 0.02 + 1
            gb = torch.randn(co, device=dev) * 0.02
            y = torch.empty((1, co) + shape[2:], dtype=dt, device=dev)
            z = torch.empty_like(y)
            cws = dit_hip._conv_ws(x, True)
            gws = torch.empty(dit_hip.load().dt_groupnorm_workspace_bytes(1, co, shape[2] * shape[3], 32),
                              dtype=torch.uint8, device=dev)
            _, stats = dit_hip.conv2d_gn(x, wp, 32, bias=b, out=y, workspace=cws)
            t_conv = time_cold(torch, lambda: dit_hip.conv2d(x, wp, bias=b, out=y, workspace=cws), reps, flush)
            t_convgn = time_cold(torch, lambda: dit_hip.conv2d_gn(x, wp, 32, bias=b, out=y, workspace=cws), reps,
                                 flush)
            t_gn2 = time_cold(torch, lambda: dit_hip.groupnorm_silu(y, 32, gw, gb, 1e-6, out=z, workspace=gws), reps,
                              flush)
            t_gn1 = time_cold(torch, lambda: dit_hip.groupnorm_silu_from_stats(y, stats, 32, gw, gb, 1e-6, out=z),
                              reps, flush)
            flop = 2.0 * co * shape[1] * 9 * shape[2] * shape[3]
            gn_bytes = 2 * y.numel() * es
            name = f"conv3x3_{shape[1]}x{shape[2]}x{shape[3]}_to_{co}_{tag}"
            out[name] = {
                "conv_us": round(t_conv * 1e6, 1), "conv_tflops": round(flop / t_conv / 1e12, 1),
                "conv_frac_mfma": round(flop / t_conv / 1e12 / MFMA_PEAK_TFLOPS, 3),
                "conv_with_gn_stats_us": round(t_convgn * 1e6, 1),
                "groupnorm_two_pass_us": round(t_gn2 * 1e6, 1),
                "groupnorm_from_stats_us": round(t_gn1 * 1e6, 1),
                "groupnorm_from_stats_frac_hbm": round(gn_bytes / t_gn1 / 1e9 / HBM_PEAK_GBS, 3),
                "conv_plus_groupnorm_us": {"two_pass": round((t_conv + t_gn2) * 1e6, 1),
                                           "stats_in_conv": round((t_convgn + t_gn1) * 1e6, 1)},
            }
            del x, y, z, cws
    return out


def cpu_baseline(budget_s):
    """The oracle's fp32 restatement of the same chain on host cores.
    Returns (GB/s-equivalent over the same algorithmic bytes, threads,
    sample description, 4-thread GB/s)."""
    import numpy as np
    sys.path.insert(0, ROOT)
    import oracle

    seed = oracle.tensor_seed
    pos = positions()
    h = oracle.round_bf16(oracle.randn(seed(0), (S, D)))
    o = oracle.round_bf16(oracle.randn(seed(1), (S, D)))
    gate = oracle.randn(seed(2), (D,), std=0.1)
    sh = oracle.randn(seed(3), (D,), std=0.1)
    sc = oracle.randn(seed(4), (D,), std=0.1)
    q = oracle.round_bf16(oracle.randn(seed(5), (S, H, HD)))
    k = oracle.round_bf16(oracle.randn(seed(6), (S, H, HD)))
    w = oracle.randn(seed(7), (HD,), mean=1.0, std=0.02)
    g = oracle.round_bf16(oracle.randn(seed(8), (S, I)))
    u = oracle.round_bf16(oracle.randn(seed(9), (S, I)))
    total = sum(alg_bytes()[0].values())

    def chain(threads):
        r = oracle.round_bf16(oracle.gated_residual(h, o, gate, threads))
        oracle.adaln(r, sh, sc, 1e-6, threads)
        oracle.qk_rmsnorm_rope(q, w, pos, 32, 10000.0, 1e-6, threads)
        oracle.qk_rmsnorm_rope(k, w, pos, 32, 10000.0, 1e-6, threads)
        oracle.swiglu(g, u, threads)

    def measure(threads, budget):
        times = []
        t_end = time.perf_counter() + budget
        chain(threads)  # warm
        while time.perf_counter() < t_end and len(times) < 200:
            t0 = time.perf_counter()
            chain(threads)
            times.append(time.perf_counter() - t0)
        return statistics.median(times), len(times)

    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    threads = max(1, min(cores, int(os.environ.get("OMP_NUM_THREADS", cores))))
    t_all, n_all = measure(threads, budget_s)
    t_4, n_4 = measure(4, budget_s / 2)
    sample = (f"full chain (gated residual, adaLN of r, QK of q and k, SwiGLU) at the GPU workload's "
              f"shape, median of {n_all} runs ({threads} threads) / {n_4} runs (4 threads, ggml's "
              f"default n_threads)")
    return total / t_all / 1e9, threads, sample, total / t_4 / 1e9


def _threads():
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    return max(1, min(cores, int(os.environ.get("OMP_NUM_THREADS", cores))))


def _median_time(fn, budget, max_runs=50):
    """Median wall time of fn() over as many runs as fit in `budget` seconds
    (at least one, after one untimed run when the budget allows)."""
    t0 = time.perf_counter()
    fn()
    first = time.perf_counter() - t0
    times = [first]
    if first * 3 < budget:
        times = []
        t_end = time.perf_counter() + budget
        while time.perf_counter() < t_end and len(times) < max_runs:
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


CFG1 = dict(n_txt=512, grid=32, dim=3072, heads=24, theta=2000.0)


def config1_inputs():
    """The single-stream block workload: 1536 tokens (512 text tokens at
    position 0, then a 32 x 32 image grid), hidden 3072, 24 x 128 heads, MLP
    9216, theta 2000; Linear weights N(0, 0.02), RMSNorm weights N(1, 0.02),
    activations N(0, 1), modulation = SiLU + Linear of a N(0, 1) vector."""
    import numpy as np
    sys.path.insert(0, ROOT)
    import oracle
    import oracle.flux2 as of
    D, heads = CFG1["dim"], CFG1["heads"]
    txt = [[0, 0, 0, 0]] * CFG1["n_txt"]
    img = [[0, y, x, 0] for y in range(CFG1["grid"]) for x in range(CFG1["grid"])]
    pos = np.array(txt + img, dtype=np.int32)
    from concurrent.futures import ThreadPoolExecutor

    def draw(item):  # one seeded stream per tensor, drawn in parallel (the C generator releases the GIL)
        i, (name, shape) = item
        seed = oracle.tensor_seed(100 + i)
        return name, (oracle.randn(seed, shape, std=0.02) if len(shape) == 2 else
                      oracle.randn(seed, shape, mean=1.0, std=0.02))
    with ThreadPoolExecutor(max_workers=8) as ex:
        P = dict(ex.map(draw, enumerate(sorted(of.single_block_param_shapes(D, heads).items()))))
    x = oracle.randn(oracle.tensor_seed(90), (pos.shape[0], D))
    cond = oracle.randn(oracle.tensor_seed(91), (1, D))
    mod = oracle.linear(of.silu(cond), oracle.randn(oracle.tensor_seed(92), (3 * D, D), std=0.02))
    return x, mod.reshape(-1), pos, P


def config1_gpu(x, mod, pos, P, dtype):
    """The same block through dit_cli Flux2SingleTransformerBlock (weights
    uploaded once and kept in HBM; inputs uploaded before each run): median
    ms per forward, or None when the driver is missing."""
    import tempfile
    import numpy as np
    cli = os.path.join(PKG, "bin", "dit_cli")
    if not os.path.exists(cli):
        return None

    def dtb(path, a, type_id):
        a = np.ascontiguousarray(a)
        with open(path, "wb") as f:
            f.write(np.array([0x31425444, type_id, a.ndim, 0], np.int32).tobytes())
            f.write(np.array(a.shape, np.int64).tobytes())
            f.write(a.tobytes())

    with tempfile.TemporaryDirectory() as d:
        wd = os.path.join(d, "w")
        os.makedirs(wd)
        for name, a in P.items():
            dtb(os.path.join(wd, name + ".dtb"), a.astype(np.float32), 0)
        S, D = x.shape
        dtb(os.path.join(d, "x.dtb"), x.reshape(1, S, D).astype(np.float32), 0)
        dtb(os.path.join(d, "mod.dtb"), mod.reshape(1, -1).astype(np.float32), 0)
        dtb(os.path.join(d, "pos.dtb"), pos, 26)
        cmd = [cli, "Flux2SingleTransformerBlock", "--heads", str(CFG1["heads"]), "--theta", str(int(CFG1["theta"]))]
        for _ in range(4):
            cmd += ["--axes_dim", "32"]
        cmd += ["--weights", wd, "--hidden_states", os.path.join(d, "x.dtb"), "--temb_mod",
                os.path.join(d, "mod.dtb"), "--position_ids", os.path.join(d, "pos.dtb"), "--dtype", dtype,
                "--out", os.path.join(d, "out.dtb"), "--resident-weights", "true", "--warmup", "3", "--steps", "10"]
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
        if r.returncode != 0:
            raise RuntimeError(f"dit_cli block failed ({r.returncode}): {r.stderr.strip()[-500:]}")
        return json.loads(r.stdout.strip().splitlines()[-1])["ms_per_compute_median"]


def cpu_configs(budget, with_gpu_block):
    """CPU baselines of the other workloads on the oracle's C restatement
    (fp32), each at all of this host's cores and at 4 threads (ggml's default
    n_threads): the single-stream block (1536 x 3072, timed beside the same
    block on the GPU), the dequantisation of the three weight matrices (Q8_0
    and Q4_K to fp32 values) and GroupNorm(32)+SiLU at the four decoder map
    shapes."""
    import numpy as np
    sys.path.insert(0, ROOT)
    import oracle
    import oracle.flux2 as of
    threads = _threads()
    out = {}

    x, mod, pos, P = config1_inputs()
    flop = 2.0 * x.shape[0] * sum(a.size for a in P.values() if a.ndim == 2) + 4.0 * x.shape[0] ** 2 * x.shape[1]
    blk = lambda t: of.single_block(x, mod, pos, P, CFG1["heads"], CFG1["theta"], 32, threads=t)
    t_all, n_all = _median_time(lambda: blk(threads), budget / 3)
    t_4, n_4 = _median_time(lambda: blk(4), budget / 3, max_runs=3)
    c1 = {"unit": "s per block forward", "value": round(t_all, 4), "cores": threads, "value_4_threads": round(t_4, 4),
          "gflop_per_forward": round(flop / 1e9, 1), "cpu_gflops": round(flop / t_all / 1e9, 1),
          "sample": f"one Flux2 single-stream block forward, fp32, 1536 tokens x 3072 (median of {n_all} runs at "
                    f"{threads} threads / {n_4} at 4 threads)"}
    if with_gpu_block:
        for dt in ("bf16", "f32"):
            ms = config1_gpu(x, mod, pos, P, dt)
            if ms is not None:
                c1[f"gpu_ms_{dt}_activations"] = round(ms, 3)
                c1[f"gpu_speedup_{dt}_vs_all_cores"] = round(t_all / (ms * 1e-3), 1)
    out["single_block_1536x3072_f32"] = c1
    del P, x

    deq = {}
    w = oracle.randn(oracle.tensor_seed(200), (3072 * 9216,), std=0.02)
    # block k covers flat elements [qk k, qk (k + 1)) for any row width that is a multiple of qk
    quant = {qt: oracle.quantize(w.reshape(-1, 3072), qt) for qt in (8, 12)}
    for rows, cols in DEQ_SHAPES:
        for tag, qt, qk, bs in (("q8_0", 8, 32, 34), ("q4_K", 12, 256, 144)):
            blocks = quant[qt][:rows * cols // qk * bs]     # the same bytes a [rows, cols] matrix quantises to
            nbytes = blocks.size + rows * cols * 2          # the GPU's bytes: blocks in, bf16 out
            y = np.zeros(rows * cols, np.float32)            # reused, as ggml reuses its buffers
            ta, _ = _median_time(lambda: oracle.dequantize(blocks, rows * cols, qt, threads, y), budget / 30)
            t4, _ = _median_time(lambda: oracle.dequantize(blocks, rows * cols, qt, 4, y), budget / 30)
            deq[f"{tag}_{rows}x{cols}"] = {"GBs": round(nbytes / ta / 1e9, 2), "GBs_4_threads": round(nbytes / t4 / 1e9, 2),
                                            "ms": round(ta * 1e3, 2)}
    out["dequant"] = {"unit": "GB/s over the GPU kernel's bytes (blocks in, bf16 out)", "cores": threads,
                      "sample": "each matrix dequantised whole to fp32 (median over ~1/30 of the budget each)",
                      "matrices": deq}

    gn = {}
    for shape in GN_SHAPES:
        xg = oracle.randn(oracle.tensor_seed(300), shape)
        wg = oracle.randn(oracle.tensor_seed(301), (shape[1],), mean=1.0, std=0.02)
        bg = oracle.randn(oracle.tensor_seed(302), (shape[1],), std=0.02)
        nbytes = 2 * xg.size * 4
        yg = np.zeros_like(xg)                               # reused, as ggml reuses its buffers
        ta, _ = _median_time(lambda: oracle.groupnorm_silu(xg, 32, wg, bg, 1e-6, True, threads, yg), budget / 16)
        t4, _ = _median_time(lambda: oracle.groupnorm_silu(xg, 32, wg, bg, 1e-6, True, 4, yg), budget / 16)
        gn["x".join(map(str, shape))] = {"GBs": round(nbytes / ta / 1e9, 2), "GBs_4_threads": round(nbytes / t4 / 1e9, 2),
                                          "ms": round(ta * 1e3, 2)}
        del xg, yg
    out["groupnorm_silu_f32"] = {"unit": "GB/s over fp32 in + out", "cores": threads,
                                 "sample": "each map normalised whole (median over ~1/16 of the budget each)",
                                 "maps": gn}
    return out


def denoise_flops(n_img=4096, n_txt=512, d=3072, mlp=9216, blocks=25, txt_width=2560, ch=128):
    """FLOP of one step: every Linear (2*M*N*K) and attention (4*S^2*d per block)."""
    s = n_img + n_txt
    per_token = 4 * d * d + 3 * d * mlp              # q, k, v, out + gate, up, down (both block types)
    lin = blocks * s * per_token
    lin += n_img * ch * d + n_txt * txt_width * d + n_img * d * ch      # x / context embedders, proj_out
    lin += 256 * d + d * d + d * (6 * d * 2 + 3 * d) + d * 2 * d        # time embedding, modulations, norm_out
    return 2 * lin + blocks * 4 * s * s * d


def denoise_step(steps, warmup, weight_format="bf16", hip_graph=True):
    """Run the full-step driver as a child process; None if it is missing.
    weight_format: what the GEMMs read, bf16 copies of the Q8_0 weights or
    the Q8_0 weights themselves (dequantised inside the GEMM).  hip_graph:
    the step's launches recorded once and replayed as one HIP graph (the
    first warm-up step runs eagerly and records), else launched one by one
    after the fusion pass every step."""
    import subprocess
    cli = os.path.join(PKG, "bin", "dit_cli")
    if not os.path.exists(cli):
        return None
    cmd = [cli, "Flux2Transformer2DModel", "--random-weights", "1", "--random-inputs", "2",
           "--steps", str(steps), "--warmup", str(warmup), "--weight-format", weight_format,
           "--hip-graph", "true" if hip_graph else "false"]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
    if r.returncode != 0:
        raise RuntimeError(f"dit_cli failed ({r.returncode}): {r.stderr.strip()[-500:]}")
    res = json.loads(r.stdout.strip().splitlines()[-1])
    if res["output"]["nonfinite"]:
        raise RuntimeError(f"denoise step output holds {res['output']['nonfinite']} non-finite values")
    t = res["ms_per_step_median"] * 1e-3
    flops = denoise_flops()
    return {
        "workload": "Flux2-klein-4B-shaped transformer step at 1024^2: 5 double + 20 single blocks, "
                    "hidden 3072, 24x128 heads, MLP 9216, 4096 image + 512 text tokens (text width 2560), "
                    "timestep 0.5, no guidance embedding",
        "weights": ("Q8_0 (N(0,0.02) quantised on device) dequantised once to bf16"
                    if weight_format == "bf16" else
                    "Q8_0 (N(0,0.02) quantised on device) kept as Q8_0 (codes + fp32 scales, 1.125 B/weight)")
                   + "; RMSNorm weights N(1,0.02)",
        "linear_weight_bytes": res["linear_weight_bytes"],
        "gemm": ("hand-written bf16 MFMA GEMM (diffusers-cpp_amd/csrc/gemm.hip"
                 + (", Q8_0 codes dequantised to bf16 as they are staged into LDS)" if weight_format == "q8_0" else ")")
                 if res.get("gemm") == "mfma" else res.get("gemm")),
        "launch": "one HIP graph replay per step" if hip_graph else "eager launches after the fusion pass",
        "s_per_step": round(t, 5),
        "ms_per_step_min": res["ms_per_step_min"],
        "ms_per_step_mean": res["ms_per_step_mean"],
        "steps": steps,
        "warmup": warmup,
        "params": res["params"],
        "graph_nodes": res["nodes"],
        "kernels_per_step": res["kernels"],
        "fused_nodes": res["fused_nodes"],
        "arena_bytes": res["arena_bytes"],
        "tflop_per_step": round(flops / 1e12, 3),
        "output": res["output"],
        "roofline": {"bound": "mfma", "achieved": round(flops / t / 1e12, 1), "peak": 2500.0,
                     "unit": "TFLOP/s", "frac": round(flops / t / 1e12 / 2500.0, 4)},
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--cpu-budget", type=float, default=12.0,
                    help="seconds of CPU-baseline sampling (0 disables)")
    ap.add_argument("--no-secondary", dest="secondary", action="store_false",
                    help="skip the dequantisation / GroupNorm measurements")
    ap.add_argument("--denoise-steps", type=int, default=5,
                    help="timed full denoising steps (0 skips the step measurement)")
    ap.add_argument("--denoise-warmup", type=int, default=2)
    ap.add_argument("--vae-only", action="store_true",
                    help="print only the VAE conv / GroupNorm measurements (one JSON line)")
    ap.add_argument("--secondary-only", action="store_true",
                    help="print only the dequantisation / GroupNorm measurements and the copy calibration "
                         "(one JSON line; the profiled workload of the dequant and GroupNorm summaries)")
    ap.add_argument("--cpu-configs-budget", type=float, default=24.0,
                    help="seconds of CPU baselines for the block, dequantisation and GroupNorm workloads "
                         "(0 disables)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this benchmark measures one GPU only (--gpus {args.gpus} requested); "
              "the chain is row-independent and would shard tokens across GPUs with no exchange",
              file=sys.stderr)
        sys.exit(2)

    if args.vae_only or args.secondary_only:
        import torch
        import dit_hip
        dit_hip.load()
        dev = torch.device("cuda:0")
        flush = Flusher(torch, dev)
        if args.vae_only:
            print(json.dumps({"vae": vae_measurements(torch, dev, flush)}), flush=True)
        else:
            print(json.dumps({"secondary": secondary(torch, dev, flush),
                              "cold_torch_copy_GBs": round(cold_torch_copy(torch, dev, flush), 1)}), flush=True)
        return

    # The CPU baselines of the other workloads run before this process
    # touches the GPU (the block's GPU timing is a child process).
    cpu_other = cpu_configs(args.cpu_configs_budget, args.denoise_steps > 0) if args.cpu_configs_budget > 0 else None

    # The full step runs in its own process before this one touches the GPU.
    denoise = denoise_step(args.denoise_steps, args.denoise_warmup) if args.denoise_steps > 0 else None
    denoise_eager = (denoise_step(args.denoise_steps, args.denoise_warmup, hip_graph=False)
                     if args.denoise_steps > 0 and args.secondary else None)
    denoise_q8 = (denoise_step(args.denoise_steps, args.denoise_warmup, "q8_0")
                  if args.denoise_steps > 0 and args.secondary else None)
    # The three runs compute the same step on the same weights and inputs:
    # graph replay, eager launches and Q8_0 weights (dequantised in the
    # GEMM's load path to the same bf16 values) must agree bit for bit.
    ref_hash = denoise["output"]["fnv64"] if denoise else None
    for name, other in (("eager launches", denoise_eager), ("Q8_0 weights", denoise_q8)):
        if other and other["output"]["fnv64"] != ref_hash:
            raise RuntimeError(f"denoise step with {name} differs from the graph-replayed bf16 step "
                               f"({other['output']} vs {denoise['output']})")

    import torch
    import dit_hip

    dit_hip.load()
    dev = torch.device("cuda:0")
    sets = [make_inputs(torch, dev, 0x5EED0000 + 97 * i) for i in range(NSETS)]
    # The launches through the Python binding's wrappers (captured into the
    # HIP graphs, which take the capturing stream), and the same launches
    # prepared once (dit_hip.prepare: the C-ABI call with its arguments
    # converted) for the eager step and the back-to-back timings, so that no
    # Python work sits between launches, as for a C++ caller.
    chain_calls = [chain_kernels(t) for t in sets]
    chains = [{k: dit_hip.prepare(f)[1] for k, f in c.items()} for c in chain_calls]

    def step(i):
        for f in chains[i % NSETS].values():
            f()

    def step_w(i):
        for f in chain_calls[i % NSETS].values():
            f()

    def warm(run_step):
        """--warmup untimed steps, continued until at least MIN_WARM_S of
        them have run: the GPU's clocks take tens of milliseconds of load to
        settle, and a short warm-up times the ramp instead of the kernels."""
        torch.cuda.synchronize()
        t0, n = time.perf_counter(), 0
        while n < args.warmup or time.perf_counter() - t0 < MIN_WARM_S:
            for _ in range(max(args.warmup, 50)):
                run_step(n)
                n += 1
            torch.cuda.synchronize()
        return n

    warm_steps = {"eager": warm(step)}
    st = torch.cuda.current_stream()

    def timed(run_step):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        w0 = time.perf_counter()
        e0.record(torch.cuda.current_stream())
        for i in range(args.steps):
            run_step(i)
        e1.record(torch.cuda.current_stream())
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3 / args.steps, time.perf_counter() - w0

    eager_s, eager_wall = timed(step)

    def capture(fn):
        """One HIP graph per buffer set of fn(i)."""
        side = torch.cuda.Stream()
        side.wait_stream(st)
        with torch.cuda.stream(side):
            for i in range(NSETS):
                fn(i)
        st.wait_stream(side)
        torch.cuda.synchronize()
        out = []
        for i in range(NSETS):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                fn(i)
            out.append(g)
        return out

    # The step's two launches captured back to back.
    graphs = capture(step_w)
    warm_steps["graph"] = warm(lambda i: graphs[i % NSETS].replay())
    seq_s, seq_wall = timed(lambda i: graphs[i % NSETS].replay())

    schedules = {"eager": eager_s, "graph": seq_s}
    best = min(schedules, key=schedules.get)
    step_s = schedules[best]
    wall = {"eager": eager_wall, "graph": seq_wall}[best]

    # The streaming ceiling: the probe launches with the chain's shapes, timed
    # the same ways (eager steps over the rotating buffer sets; cold launches).
    probes = [probe_kernels(t) for t in sets]

    def probe_step(i):
        for f in probes[i % NSETS].values():
            f()

    warm(probe_step)
    probe_s, _ = timed(probe_step)

    # Block order with the four standalone kernels, as a graph, for comparison.
    single_calls = [standalone_kernels(t) for t in sets]
    singles = [{k: dit_hip.prepare(f)[1] for k, f in c.items()} for c in single_calls]

    def unfused(i):
        for f in single_calls[i % NSETS].values():
            f()

    ugraphs = capture(unfused)
    warm(lambda i: ugraphs[i % NSETS].replay())
    unfused_s, _ = timed(lambda i: ugraphs[i % NSETS].replay())
    del graphs, ugraphs

    fused_ab, single_ab = alg_bytes()
    total = sum(fused_ab.values())
    flush = Flusher(torch, dev)

    def cold(fns, ab):
        res = {}
        for name, fn in fns.items():
            ts = time_cold(torch, fn, 20, flush, samples=True)
            tk = statistics.median(ts)
            res[name] = {"us": round(tk * 1e6, 2), "us_mean": round(statistics.mean(ts) * 1e6, 2),
                         "us_min": round(min(ts) * 1e6, 2), "alg_MB": round(ab[name] / 1e6, 2),
                         "GBs": round(ab[name] / tk / 1e9, 1),
                         "frac_hbm": round(ab[name] / tk / 1e9 / HBM_PEAK_GBS, 3)}
        return res

    kernels = cold(chains[0], fused_ab)
    # Each launch alone, back to back over the buffer sets (HIP events around
    # the run): its average duration inside a stream of launches.
    for name in kernels:
        ts = time_stream(torch, [c[name] for c in chains], 40 * NSETS)
        kernels[name]["us_stream_mean"] = round(ts * 1e6, 2)
        kernels[name]["GBs_stream"] = round(fused_ab[name] / ts / 1e9, 1)
        kernels[name]["frac_hbm_stream"] = round(fused_ab[name] / ts / 1e9 / HBM_PEAK_GBS, 4)
    probe_cold = {name: time_cold(torch, fn, 20, flush) for name, fn in probes[0].items()}
    for name, k in kernels.items():
        k["stream_probe_us"] = round(probe_cold[name] * 1e6, 2)
        k["frac_of_stream_probe"] = round(probe_cold[name] * 1e6 / k["us"], 3)
    kernels_standalone = cold(singles[0], single_ab)
    for name in kernels_standalone:
        ts = time_stream(torch, [c[name] for c in singles], 40 * NSETS)
        kernels_standalone[name]["us_stream_mean"] = round(ts * 1e6, 2)
        kernels_standalone[name]["frac_hbm_stream"] = round(single_ab[name] / ts / 1e9 / HBM_PEAK_GBS, 4)
    cold_copy = cold_torch_copy(torch, dev, flush)
    extra = secondary(torch, dev, flush) if args.secondary else None
    if extra is not None:
        extra["vae"] = vae_measurements(torch, dev, flush)

    dom = "qk_swiglu"
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "qk_swiglu_4608_bf16_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("bytes_per_launch")
    kd = kernels[dom]
    roofline = {"bound": "hbm", "achieved": kd["GBs_stream"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(kd["GBs_stream"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                "kernel": "qk_swiglu_kernel<bf16,3,1>", "alg_bytes_per_launch": fused_ab[dom],
                "statistic": f"mean launch duration over {40 * NSETS} back-to-back launches cycling {NSETS} buffer "
                             f"sets (HIP events around the run, on the launch stream)",
                "launch_us_stream_mean": kd["us_stream_mean"],
                "single_cold_launch_us": {"median": kd["us"], "mean": kd["us_mean"], "min": kd["us_min"],
                                          "statistic": "20 launches, each bracketed by HIP events after a "
                                                       "1 GiB cache flush (adds the dispatch latency)"},
                "frac_single_cold_median": round(kd["GBs"] / HBM_PEAK_GBS, 4)}

    cpu = None
    if args.cpu_budget > 0:
        v, cores, sample, v4 = cpu_baseline(args.cpu_budget)
        cpu = {"value": round(v, 2), "unit": "GB/s", "cores": cores, "kind": "port",
               "sample": sample, "value_4_threads": round(v4, 2)}
        if cpu_other:
            cpu["other_workloads"] = cpu_other

    value = total / step_s / 1e9
    out = {
        "metric": "fused DiT elementwise GB/s (% HBM peak); sec/denoise step at 1024² on 1 GPU",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_steps_run": warm_steps,
        "ms_per_step": round(step_s * 1e3, 4),
        "schedule": best,
        "schedules_ms_per_step": {k: round(v * 1e3, 4) for k, v in schedules.items()},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.1) modulation vectors)",
        "config": {"workload": "Flux2 single-stream block elementwise chain, bf16, two fused launches: "
                               "gated residual + adaLN h,o[4608,3072] -> r,y; QK-RMSNorm+4-axis RoPE "
                               "q,k[4608,24,128] + SwiGLU [4608,18432]->[4608,9216]",
                   "alg_bytes_per_step": total, "buffer_sets": NSETS,
                   "parallelism": "none (1 GPU)"},
        "unfused_graph_ms_per_step": round(unfused_s * 1e3, 4),
        "unfused_alg_bytes_per_step": sum(single_ab.values()),
        "frac_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        "sec_per_denoise_step": denoise["s_per_step"] if denoise else None,
        "denoise_step": denoise,
        "denoise_step_q8_0_weights": denoise_q8,
        "denoise_step_eager_launches": denoise_eager,
        "cold_torch_copy_GBs": round(cold_copy, 1),
        "stream_probe_ms_per_step": round(probe_s * 1e3, 4),
        "stream_probe_GBs": round(total / probe_s / 1e9, 1),
        "frac_of_stream_probe": round(probe_s / step_s, 4),
        "kernels": kernels,
        "kernels_standalone": kernels_standalone,
        "secondary": extra,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "wall_s_timed_region": round(wall, 4) if wall else None,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
