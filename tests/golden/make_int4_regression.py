"""Writes tests/golden/int4_one_launch_M1_K512_N384_E8_k2.npz: a regression pin
of the single-token tiled-int4 route (one fused GEMM1 + activation + GEMM2
launch and the fixed-order plane sum), run on the GPU.

The product's own output is stored, not an oracle's: the oracle check of the
same route (tests/test_int4_tiled.py) is at the int4 tolerance, which a small
change of the summation order would pass unnoticed.  This pin catches such a
change bit for bit; regenerate it only for a deliberate change of the route's
arithmetic.  Inputs follow the oracle's seeded recipe (CPU torch generator)
and are checked by SHA-256.

Run from the repo root on a GPU box:  python tests/golden/make_int4_regression.py
"""

import hashlib
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
for p in (ROOT, os.path.join(ROOT, "flaggems-sglang_amd")):
    sys.path.insert(0, p)

SHAPE = (1, 512, 384, 8, 2)  # M, K, N, E, k
NAME = "int4_one_launch_M{}_K{}_N{}_E{}_k{}.npz".format(*SHAPE)


def run_case():
    """(input SHA-256, output bf16 bits) of the one-launch route on cuda."""
    import flaggems_sglang
    from flaggems_sglang import quant as Q
    from oracle import fused_moe_oracle as O

    M, K, N, E, k = SHAPE
    d = O.make_inputs(M, K, N, E, k, wscale=0.05)
    h = hashlib.sha256()
    for n in ("x", "w13", "w2", "topk_weights", "topk_ids"):
        h.update(d[n].contiguous().view(torch.uint8).numpy().tobytes())
    dev = "cuda"
    q1, s1, z1 = Q.quantize_int4_group(d["w13"].to(dev))
    q2, s2, z2 = Q.quantize_int4_group(d["w2"].to(dev))
    out = flaggems_sglang.fused_experts(
        d["x"].to(dev), Q.tile_int4(q1), Q.tile_int4(q2), d["topk_weights"].to(dev),
        d["topk_ids"].to(dev), use_int4_w4a16=True, w1_scale=s1, w2_scale=s2, w1_zp=z1, w2_zp=z2)
    bits = out.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
    return h.hexdigest(), bits


if __name__ == "__main__":
    sha, bits = run_case()
    np.savez(os.path.join(os.path.dirname(os.path.abspath(__file__)), NAME), out=bits,
             input_sha256=np.array(sha))
    print("wrote", NAME, bits.shape)
