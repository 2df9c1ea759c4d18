"""Single-pass GroupNorm + SiLU probe (gn_single_pass.hip) beside the
library's two-pass GroupNorm, on the VAE decoder's [1,512,128,128] map, fp32
and bf16 (the larger decoder maps do not fit one resident grid at up to 16
vectors per thread: the probe reports -1 for them).

    python diffusers-cpp_amd/probe/gn_single_pass.py          # check and time
    python diffusers-cpp_amd/probe/gn_single_pass.py prof     # 20 launches of each, for rocprofv3

Each single-pass output is checked against the two-pass output (the two
differ only in how the group statistics are summed).  Timing: the median of
10 launches each after a 1 GiB cache flush ("cold"), and 20 launches back to
back on the same buffers."""
import ctypes
import os
import statistics
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
sys.path.insert(0, PKG)

import torch  # noqa: E402

import dit_hip  # noqa: E402

MAPS = [(1, 512, 128, 128), (1, 512, 256, 256)]
G = 32


def main():
    prof = len(sys.argv) > 1 and sys.argv[1] == "prof"
    dit_hip.load()
    lib = ctypes.CDLL(os.path.join(PKG, "lib", "libdit_probe_gn.so"))
    f = lib.dt_probe_gn_single_pass
    f.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int64] * 4 + [ctypes.c_float, ctypes.c_int, ctypes.c_int,
                                                                 ctypes.c_int, ctypes.c_void_p, ctypes.c_int64,
                                                                 ctypes.c_void_p]
    f.restype = ctypes.c_int
    wsb = lib.dt_probe_gn_single_pass_workspace_bytes
    wsb.argtypes = [ctypes.c_int64] * 4
    wsb.restype = ctypes.c_int64
    dev = torch.device("cuda")
    flush_buf = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    for shape in MAPS:
        N, C, H, W = shape
        for dt, io in ((torch.bfloat16, 1), (torch.float32, 0)):
            torch.manual_seed(0)
            x = torch.randn(shape, device=dev).to(dt)
            w = torch.randn(C, device=dev) * 0.02 + 1
            b = torch.randn(C, device=dev) * 0.02
            y = torch.empty_like(x)
            ws = torch.zeros(wsb(N, C, H * W, G), dtype=torch.uint8, device=dev)
            ws2 = torch.empty(dit_hip.load().dt_groupnorm_workspace_bytes(N, C, H * W, G), dtype=torch.uint8,
                              device=dev)
            ref = dit_hip.groupnorm_silu(x, G, w, b, 1e-6, workspace=ws2)
            err_at = N * G * 128

            def single(form):
                return lambda: f(x.data_ptr(), y.data_ptr(), w.data_ptr(), b.data_ptr(), N, C, H * W, G, 1e-6, 1,
                                 io, form, ws.data_ptr(), ws.numel(), None)

            fns = {"single pass, relaxed device-scope barrier": single(1),
                   "single pass, acquire/release barrier": single(0),
                   "two passes (the library)": lambda: dit_hip.groupnorm_silu(x, G, w, b, 1e-6, out=y,
                                                                              workspace=ws2)}
            name = f"{'x'.join(map(str, shape))} {str(dt)[6:]}"
            for form in (1, 0):
                blocks = single(form)()
                torch.cuda.synchronize()
                if blocks == -1:
                    print(f"{name}: the grid does not fit the device at once", flush=True)
                    break
                err = int(ws[err_at:err_at + 4].view(torch.int32).item())
                rel = ((y.float() - ref.float()).norm() / ref.float().norm()).item()
                print(f"{name}: form {form}: {blocks} workgroups, wait error {err}, rel L2 to the two passes "
                      f"{rel:.2e}", flush=True)
                if blocks <= 0 or err != 0 or not rel < 1e-3:
                    sys.exit(1)
            if blocks == -1:
                continue
            if prof:
                for fn in fns.values():
                    for _ in range(20):
                        fn()
                torch.cuda.synchronize()
                continue
            for label, fn in fns.items():
                cold = []
                for _ in range(10):
                    flush_buf.fill_(len(cold) & 0xFF)
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record()
                    fn()
                    e1.record()
                    torch.cuda.synchronize()
                    cold.append(e0.elapsed_time(e1) * 1e3)
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(20):
                    fn()
                e1.record()
                torch.cuda.synchronize()
                print(f"  {label:44s} cold {statistics.median(cold):7.2f} us   back to back "
                      f"{e0.elapsed_time(e1) * 1e3 / 20:7.2f} us", flush=True)


if __name__ == "__main__":
    main()
