"""Benchmark of the fused Flux2 DiT elementwise chain on one MI355X.

Workload (one "step" = one pass of the chain over one synthetic batch, all
inputs resident in HBM, bf16 activations, fp32 math):
  adaLN            x[4608, 3072] -> (1 + scale) * LayerNorm(x) + shift
  QK-RMSNorm+RoPE  q, k [4608, 24, 128], 4 axes x 32 dims, theta 1e4,
                   positions: 512 text tokens [0,0,0,l] then a 64x64 image grid
  SwiGLU           gate | up = [4608, 18432] -> [4608, 9216]
  gated residual   h + gate * o, [4608, 3072]
Algorithmic bytes per step: every distinct input read once and every output
written once at its I/O dtype (broadcast vectors and tables counted once).

Timed steps rotate through NSETS independent buffer sets (about 1.9 GB in
all, far above the 256 MB last-level cache), so every step reads its inputs
from HBM.  Three schedules of the same step are timed: eager launches, a
HIP graph of the four launches, and a HIP graph whose independent launches
(adaLN, QK, SwiGLU) sit on parallel branches with the gated residual joined
after adaLN; `value` = whole-step algorithmic GB/s of the fastest (all
three are reported).  `roofline` is the
dominant kernel (SwiGLU) timed alone with HIP events on the stream it is
launched on; `cpu_baseline` is the oracle's C restatement of the same chain
(fp32, OpenMP) on a bounded sample, timed on this host's cores.

`sec_per_denoise_step` is one full Flux2-klein-4B-shaped transformer step
(5 double + 20 single blocks, hidden 3072, 24x128 heads, 4096 image tokens of
128 features + 512 text tokens of width 2560, timestep 0.5) run by the C++
driver (diffusers-cpp_amd/bin/dit_cli) as a child process: Q8_0 weights
drawn N(0, 0.02) and dequantised once to bf16, bf16 activations, inputs and
weights resident in HBM, median wall time per step of the recorded graph.

Prints ONE JSON line.
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "diffusers-cpp_amd")
sys.path.insert(0, PKG)

HBM_PEAK_GBS = 8000.0
NSETS = 4
S, D, H, HD, I = 4608, 3072, 24, 128, 9216
N_TXT, GRID = 512, 64


def alg_bytes():
    e = 2  # bf16
    ad = 2 * S * D * e + 2 * D * 4                 # x in, y out, shift/scale fp32
    qk = 4 * S * H * HD * e + 2 * HD * 4 + S * 4 * 4 + 512 * 32 * 4  # q,k in/out, w, pos, table
    sw = 3 * S * I * e                              # gate, up in; out
    gr = 3 * S * D * e + D * 4                      # h, o in; y out; gate
    return {"adaln": ad, "qk_rmsnorm_rope": qk, "swiglu": sw, "gated_residual": gr}


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
        "x": rn((S, D)), "shift": rn((D,), 0.1, dtype=torch.float32),
        "scale": rn((D,), 0.1, dtype=torch.float32),
        "q": rn((S, H, HD)), "k": rn((S, H, HD)),
        "wq": rn((HD,), 0.02, 1.0, torch.float32), "wk": rn((HD,), 0.02, 1.0, torch.float32),
        "pos": pos, "table": dit_hip.rope_table(N_TXT, 32, 10000.0, device=dev),
        "gu": rn((S, 2 * I)), "h": rn((S, D)), "gate": rn((D,), 0.1, dtype=torch.float32),
        "y": torch.empty((S, D), dtype=torch.bfloat16, device=dev),
        "qo": torch.empty((S, H, HD), dtype=torch.bfloat16, device=dev),
        "ko": torch.empty((S, H, HD), dtype=torch.bfloat16, device=dev),
        "sw": torch.empty((S, I), dtype=torch.bfloat16, device=dev),
        "r": torch.empty((S, D), dtype=torch.bfloat16, device=dev),
    }


def chain_kernels(t):
    import dit_hip
    gu = t["gu"]
    return {
        "adaln": lambda: dit_hip.adaln_mod(t["x"], t["shift"], t["scale"], 1e-6, out=t["y"]),
        "qk_rmsnorm_rope": lambda: dit_hip.qk_rmsnorm_rope(
            t["q"], t["k"], t["wq"], t["wk"], t["pos"], 32, 10000.0, 1e-6, table=t["table"],
            q_out=t["qo"], k_out=t["ko"]),
        "swiglu": lambda: dit_hip.swiglu(gu[:, :I], gu[:, I:], out=t["sw"]),
        # o = the adaLN output (any [S, D] bf16 activation)
        "gated_residual": lambda: dit_hip.gated_residual(t["h"], t["y"], t["gate"], out=t["r"]),
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


def time_cold(torch, fn, n, flush):
    """Median duration of fn() over n launches, each bracketed by its own HIP
    events on the launch stream, with the cache flushed before (outside) each
    bracket."""
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
    return statistics.median(a.elapsed_time(b) for a, b in ev) * 1e-3


def copy_ceiling(torch, dev, flush):
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    src.fill_(1)
    t = time_cold(torch, lambda: dst.copy_(src), 10, flush)
    return 2 * src.numel() / t / 1e9


def secondary(torch, dev, flush):
    """Configs measured beside the chain: weight dequantisation (3072x9216,
    Q8_0 and Q4_K -> bf16) and the VAE GroupNorm(32)+SiLU shapes."""
    import dit_hip
    out = {}
    rows, cols = 3072, 9216
    for name, qt, qk, bs in (("dequant_q8_0_3072x9216_bf16", dit_hip.Q8_0, 32, 34),
                             ("dequant_q4_K_3072x9216_bf16", dit_hip.Q4_K, 256, 144)):
        src = torch.randint(0, 256, (rows * cols // qk * bs,), dtype=torch.uint8, device=dev)
        view = src.view(-1, bs)
        view[:, 1] &= 0x3B                    # keep fp16 scales finite
        if qt == dit_hip.Q4_K:
            view[:, 3] &= 0x3B
        y = torch.empty((rows, cols), dtype=torch.bfloat16, device=dev)
        t = time_cold(torch, lambda: dit_hip.dequant(src, qt, rows, cols, out=y), 10, flush)
        nbytes = src.numel() + y.numel() * 2
        out[name] = {"us": round(t * 1e6, 2), "alg_MB": round(nbytes / 1e6, 2),
                     "GBs": round(nbytes / t / 1e9, 1), "frac_hbm": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 3)}
    for shape in ((1, 512, 128, 128), (1, 512, 256, 256), (1, 256, 512, 512), (1, 128, 1024, 1024)):
        for dt, es in ((torch.float32, 4), (torch.bfloat16, 2)):
            x = torch.randn(shape, device=dev).to(dt)
            w = torch.randn(shape[1], device=dev) * 0.02 + 1
            b = torch.randn(shape[1], device=dev) * 0.02
            y = torch.empty_like(x)
            ws = torch.empty(dit_hip.load().dt_groupnorm_workspace_bytes(1, shape[1], shape[2] * shape[3], 32),
                             dtype=torch.uint8, device=dev)
            t = time_cold(torch, lambda: dit_hip.groupnorm_silu(x, 32, w, b, 1e-6, out=y, workspace=ws), 6, flush)
            nbytes = 2 * x.numel() * es
            name = "groupnorm_silu_" + "x".join(map(str, shape)) + ("_f32" if es == 4 else "_bf16")
            out[name] = {"us": round(t * 1e6, 2), "alg_MB": round(nbytes / 1e6, 2),
                         "GBs": round(nbytes / t / 1e9, 1), "frac_hbm": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 3)}
            del x, y
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
    x = oracle.round_bf16(oracle.randn(seed(0), (S, D)))
    sh = oracle.randn(seed(1), (D,), std=0.1)
    sc = oracle.randn(seed(2), (D,), std=0.1)
    q = oracle.round_bf16(oracle.randn(seed(3), (S, H, HD)))
    k = oracle.round_bf16(oracle.randn(seed(4), (S, H, HD)))
    w = oracle.randn(seed(5), (HD,), mean=1.0, std=0.02)
    g = oracle.round_bf16(oracle.randn(seed(6), (S, I)))
    u = oracle.round_bf16(oracle.randn(seed(7), (S, I)))
    h = oracle.round_bf16(oracle.randn(seed(8), (S, D)))
    gate = oracle.randn(seed(9), (D,), std=0.1)
    total = sum(alg_bytes().values())

    def chain(threads):
        y = oracle.adaln(x, sh, sc, 1e-6, threads)
        oracle.qk_rmsnorm_rope(q, w, pos, 32, 10000.0, 1e-6, threads)
        oracle.qk_rmsnorm_rope(k, w, pos, 32, 10000.0, 1e-6, threads)
        oracle.swiglu(g, u, threads)
        oracle.gated_residual(h, y, gate, threads)

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
    sample = (f"full chain at the GPU workload's shape, median of {n_all} runs "
              f"({threads} threads) / {n_4} runs (4 threads, ggml's default n_threads)")
    return total / t_all / 1e9, threads, sample, total / t_4 / 1e9


def denoise_flops(n_img=4096, n_txt=512, d=3072, mlp=9216, blocks=25, txt_width=2560, ch=128):
    """FLOP of one step: every Linear (2*M*N*K) and attention (4*S^2*d per block)."""
    s = n_img + n_txt
    per_token = 4 * d * d + 3 * d * mlp              # q, k, v, out + gate, up, down (both block types)
    lin = blocks * s * per_token
    lin += n_img * ch * d + n_txt * txt_width * d + n_img * d * ch      # x / context embedders, proj_out
    lin += 256 * d + d * d + d * (6 * d * 2 + 3 * d) + d * 2 * d        # time embedding, modulations, norm_out
    return 2 * lin + blocks * 4 * s * s * d


def denoise_step(steps, warmup):
    """Run the full-step driver as a child process; None if it is missing."""
    import subprocess
    cli = os.path.join(PKG, "bin", "dit_cli")
    if not os.path.exists(cli):
        return None
    cmd = [cli, "Flux2Transformer2DModel", "--random-weights", "1", "--random-inputs", "2",
           "--steps", str(steps), "--warmup", str(warmup)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
    if r.returncode != 0:
        raise RuntimeError(f"dit_cli failed ({r.returncode}): {r.stderr.strip()[-500:]}")
    res = json.loads(r.stdout.strip().splitlines()[-1])
    t = res["ms_per_step_median"] * 1e-3
    flops = denoise_flops()
    return {
        "workload": "Flux2-klein-4B-shaped transformer step at 1024^2: 5 double + 20 single blocks, "
                    "hidden 3072, 24x128 heads, MLP 9216, 4096 image + 512 text tokens (text width 2560), "
                    "timestep 0.5, no guidance embedding",
        "weights": "Q8_0 (N(0,0.02) quantised on device) dequantised once to bf16; RMSNorm weights N(1,0.02)",
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
        "roofline": {"bound": "mfma", "achieved": round(flops / t / 1e12, 1), "peak": 2500.0,
                     "unit": "TFLOP/s", "frac": round(flops / t / 1e12 / 2500.0, 4)},
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-budget", type=float, default=12.0,
                    help="seconds of CPU-baseline sampling (0 disables)")
    ap.add_argument("--no-secondary", dest="secondary", action="store_false",
                    help="skip the dequantisation / GroupNorm measurements")
    ap.add_argument("--denoise-steps", type=int, default=5,
                    help="timed full denoising steps (0 skips the step measurement)")
    ap.add_argument("--denoise-warmup", type=int, default=2)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "the chain is row-independent and would shard tokens across GPUs with no exchange",
              file=sys.stderr)
        sys.exit(2)

    # The full step runs in its own process before this one touches the GPU.
    denoise = denoise_step(args.denoise_steps, args.denoise_warmup) if args.denoise_steps > 0 else None

    import torch
    import dit_hip

    dit_hip.load()
    dev = torch.device("cuda:0")
    sets = [make_inputs(torch, dev, 0x5EED0000 + 97 * i) for i in range(NSETS)]
    chains = [chain_kernels(t) for t in sets]

    def step(i):
        for f in chains[i % NSETS].values():
            f()

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
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

    eager_s, _ = timed(step)

    # One captured graph per buffer set: the four launches of a step.
    graphs = []
    side = torch.cuda.Stream()
    side.wait_stream(st)
    with torch.cuda.stream(side):
        for i in range(NSETS):
            step(i)
    st.wait_stream(side)
    torch.cuda.synchronize()
    for i in range(NSETS):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step(i)
        graphs.append(g)
    for i in range(args.warmup):
        graphs[i % NSETS].replay()
    seq_s, seq_wall = timed(lambda i: graphs[i % NSETS].replay())

    # The same step as a graph with parallel branches: adaLN, QK and SwiGLU
    # are independent; the gated residual consumes the adaLN output.
    def branched(i):
        c = chains[i % NSETS]
        main = torch.cuda.current_stream()
        s1, s2 = branch_streams
        s1.wait_stream(main)
        s2.wait_stream(main)
        with torch.cuda.stream(s1):
            c["qk_rmsnorm_rope"]()
        with torch.cuda.stream(s2):
            c["swiglu"]()
        c["adaln"]()
        c["gated_residual"]()
        main.wait_stream(s1)
        main.wait_stream(s2)

    branch_streams = (torch.cuda.Stream(), torch.cuda.Stream())
    bgraphs = []
    for i in range(NSETS):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            branched(i)
        bgraphs.append(g)
    for i in range(args.warmup):
        bgraphs[i % NSETS].replay()
    br_s, br_wall = timed(lambda i: bgraphs[i % NSETS].replay())
    schedules = {"eager": eager_s, "graph": seq_s, "graph_branched": br_s}
    best = min(schedules, key=schedules.get)
    step_s = schedules[best]
    wall = {"eager": None, "graph": seq_wall, "graph_branched": br_wall}[best]

    ab = alg_bytes()
    total = sum(ab.values())
    flush = Flusher(torch, dev)
    kernels = {}
    for name in chains[0]:
        tk = time_cold(torch, chains[0][name], 20, flush)
        kernels[name] = {"us": round(tk * 1e6, 2), "alg_MB": round(ab[name] / 1e6, 2),
                         "GBs": round(ab[name] / tk / 1e9, 1),
                         "frac_hbm": round(ab[name] / tk / 1e9 / HBM_PEAK_GBS, 3)}
    ceiling = copy_ceiling(torch, dev, flush)
    extra = secondary(torch, dev, flush) if args.secondary else None

    dom = "swiglu"
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "swiglu_4608x9216_bf16_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("bytes_per_launch")
    roofline = {"bound": "hbm", "achieved": kernels[dom]["GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(kernels[dom]["GBs"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                "kernel": "swiglu_kernel<bf16,2>", "alg_bytes_per_launch": ab[dom]}

    cpu = None
    if args.cpu_budget > 0:
        v, cores, sample, v4 = cpu_baseline(args.cpu_budget)
        cpu = {"value": round(v, 2), "unit": "GB/s", "cores": cores, "kind": "port",
               "sample": sample, "value_4_threads": round(v4, 2)}

    value = total / step_s / 1e9
    out = {
        "metric": "fused DiT elementwise GB/s (% HBM peak); sec/denoise step at 1024² on 1 GPU",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_s * 1e3, 4),
        "schedule": best,
        "schedules_ms_per_step": {k: round(v * 1e3, 4) for k, v in schedules.items()},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.1) modulation vectors)",
        "config": {"workload": "Flux2 DiT elementwise chain, bf16: adaLN x[4608,3072] + "
                               "QK-RMSNorm+4-axis RoPE q,k[4608,24,128] + SwiGLU [4608,18432]->"
                               "[4608,9216] + gated residual [4608,3072]",
                   "alg_bytes_per_step": total, "buffer_sets": NSETS,
                   "parallelism": "none (1 GPU)"},
        "frac_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        "sec_per_denoise_step": denoise["s_per_step"] if denoise else None,
        "denoise_step": denoise,
        "copy_ceiling_GBs": round(ceiling, 1),
        "kernels": kernels,
        "secondary": extra,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "wall_s_timed_region": round(wall, 4) if wall else None,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
