"""Writes tests/golden/flux2_full_step_1024.npz: the oracle's output of the
full Flux2-klein-4B-shaped transformer at 1024^2 (Flux2Transformer2DModel::
forward, src/diffusers/models/transformers/flux2/Flux2Transformer2DModel.cpp:
111-231): 5 double + 20 single blocks, hidden 3072, 24 x 128 heads, MLP 9216,
4096 image tokens (a 64 x 64 grid of 128 features) + 512 text tokens of width
2560, theta 2000, timestep 0.5.

Weights are the ones dit_cli --hash-weights 11 draws (Q8_0 blocks by the
integer rule oracle.c states, regenerated here bit for bit); inputs are
oracle.randn draws rounded to bf16, seeds below.  Two outputs:
  exact  -- the model multiplying by the exact Q8_0 values in fp32;
  ggml   -- the same with ggml's CPU Q8_0 arithmetic in every Linear
            (activations quantised to Q8_0), the reference's own arithmetic.
The full step is ~40 TFLOP on the host cores (minutes), too slow for a GPU
test to recompute, so the GPU test compares against these stored outputs.

Run: python tests/golden/make_full_step.py  (from the repository root)
"""
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle as orc  # noqa: E402
import oracle.flux2 as of  # noqa: E402

CFG = dict(num_layers=5, num_single_layers=20, num_attention_heads=24, attention_head_dim=128,
           in_channels=128, joint_attention_dim=2560, timestep_guidance_channels=256, mlp_ratio=3.0,
           rope_theta=2000, axes_dims_rope=[32, 32, 32, 32], eps=1e-6)
N_TXT, GRID, HASH_SEED, TIMESTEP = 512, 64, 11, 0.5
HIDDEN_SEED, TEXT_SEED = 9990, 9991
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "flux2_full_step_1024.npz")


def positions(n_txt, grid):
    """Text token l at (0, 0, 0, l); image token (y, x) at (0, y, x, 0)."""
    txt = np.array([[0, 0, 0, l] for l in range(n_txt)], dtype=np.int32)
    img = np.array([[0, y, x, 0] for y in range(grid) for x in range(grid)], dtype=np.int32)
    return np.concatenate([txt, img]).reshape(-1, 4)


def inputs():
    n_img = GRID * GRID
    hid = orc.round_bf16(orc.randn(orc.tensor_seed(HIDDEN_SEED), (n_img, CFG["in_channels"])))
    txt = orc.round_bf16(orc.randn(orc.tensor_seed(TEXT_SEED), (N_TXT, CFG["joint_attention_dim"])))
    return hid, txt, positions(N_TXT, GRID)


class HashParams:
    """Parameters as dit_cli --hash-weights draws them (see the GPU test's
    class of the same name): exact fp32 values, or Q8_0Weight blocks."""

    def __init__(self, seed, shapes, exact):
        self.seed, self.shapes, self.exact = seed, shapes, exact

    def __getitem__(self, name):
        shape = self.shapes[name]
        if len(shape) == 1:
            return orc.hash_norm_weight(self.seed, name, shape[0])
        rows, cols = shape
        w = orc.Q8_0Weight(orc.hash_q8_0(self.seed, name, rows, cols), rows, cols)
        return w.dequantize() if self.exact else w


def main():
    hid, txt, pos = inputs()
    shapes = of.model_param_shapes(CFG)
    outs = {}
    for name, exact in (("exact", True), ("ggml", False)):
        t0 = time.time()
        outs[name] = of.model(hid, txt, TIMESTEP, pos[N_TXT:], pos[:N_TXT], HashParams(HASH_SEED, shapes, exact),
                              CFG)
        print(f"{name}: {time.time() - t0:.1f} s, std {outs[name].std():.4f}", flush=True)
    np.savez(OUT, exact=outs["exact"], ggml=outs["ggml"],
             meta=np.array([N_TXT, GRID, HASH_SEED, HIDDEN_SEED, TEXT_SEED], np.int64),
             timestep=np.array([TIMESTEP], np.float32))
    print("wrote", OUT)


if __name__ == "__main__":
    main()
