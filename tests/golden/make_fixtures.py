"""Writes the golden fixtures of the fused-MoE path (tests/golden/*.npz).

The reference holds no golden vectors for this path (its tests compare
against SGLang live on a GPU), so these are produced by the CPU oracle
(oracle/fused_moe_oracle.py) on the reference's own input recipe
(tests/test_fused_moe.py:50-58: x ~ N(0,1), weights N(0,1)*0.1, softmax top-k,
seed M+K+N+E+topk) at the reference's FUSED_MOE_SHAPES_SMALL
(tests/accuracy_utils.py:100-102), the BASELINE tiny config, and small
fp8 / int4 / activation / bias cases.

To keep the files small, large inputs are not stored: they are regenerated
from the seeded recipe (``inputs_for`` below, also used by the tests) and
checked against the SHA-256 of their bytes stored here, so a drifting
generator fails loudly instead of silently changing the inputs.  Routing
arrays, quantized activations and every output are stored (bf16 as uint16
bits, fp8 as uint8 bits).

Run from the repo root:  python tests/golden/make_fixtures.py
"""

import hashlib
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import fused_moe_oracle as O  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
REF_SHAPES = [(1, 128, 256, 8, 2), (7, 128, 256, 8, 2), (33, 256, 512, 16, 4)]


def b16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def sha(*ts):
    h = hashlib.sha256()
    for t in ts:
        h.update(t.contiguous().view(torch.uint8).numpy().tobytes() if isinstance(t, torch.Tensor)
                 else np.ascontiguousarray(t).tobytes())
    return np.frombuffer(h.digest(), dtype=np.uint8)


def ref_inputs(M, K, N, E, topk):
    """tests/test_fused_moe.py:50-58 on CPU (w1 [E,K,2N], w2 [E,N,K])."""
    torch.manual_seed(M + K + N + E + topk)
    x = torch.randn(M, K, dtype=torch.bfloat16)
    w1 = torch.randn(E, K, N * 2, dtype=torch.bfloat16) * 0.1
    w2 = torch.randn(E, N, K, dtype=torch.bfloat16) * 0.1
    logits = torch.randn(M, E, dtype=torch.float32)
    tw, ti = O.softmax_topk(logits, topk)
    return x, w1, w2, logits, tw, ti


def inputs_for(name):
    """Regenerates the inputs of fixture ``name`` (same recipe as below)."""
    if name.startswith("ref_"):
        M, K, N, E, k = [int(v[1:]) for v in name[4:].split("_")]
        return ref_inputs(M, K, N, E, k)
    if name.startswith("tiny_"):
        return O.make_inputs(64, 128, 256, 8, 2, wscale=0.02)
    if name.startswith("quant_"):
        return O.make_inputs(5, 256, 128, 4, 2, wscale=0.02)
    if name.startswith("bias_"):
        d = O.make_inputs(6, 128, 128, 4, 2, wscale=0.1)
        g = torch.Generator().manual_seed(7)
        d["b13"] = torch.randn(4, 256, generator=g) * 0.1
        d["b2"] = torch.randn(4, 128, generator=g) * 0.1
        return d
    raise KeyError(name)


def main():
    for (M, K, N, E, topk) in REF_SHAPES:
        name = f"ref_M{M}_K{K}_N{N}_E{E}_k{topk}"
        x, w1, w2, logits, tw, ti = inputs_for(name)
        r = O.standard_topk_to_routing(tw, ti, E)
        al = O.moe_align_block_size(ti, 16, E)
        out = O.fused_experts(x, w1.transpose(1, 2), w2.transpose(1, 2), tw, ti)
        out_in = O.fused_experts(x, w1.transpose(1, 2), w2.transpose(1, 2), tw, ti,
                                 apply_router_weight_on_input=True)
        np.savez_compressed(
            os.path.join(OUT, name + ".npz"), inputs_sha256=sha(x, w1, w2, logits),
            topk_weights=tw.numpy(), topk_ids=ti.numpy().astype(np.int32),
            topk_indx=r["topk_indx"].astype(np.int32), gate_indx=r["gate_indx"].astype(np.int32),
            gate_scal=r["gate_scal"].astype(np.float32), hist=r["hist"].astype(np.int32),
            sorted_token_ids=al["sorted_token_ids"], expert_ids=al["expert_ids"],
            num_tokens_post_padded=np.asarray(al["num_tokens_post_padded"], dtype=np.int32).reshape(-1),
            out=b16(out), out_input_gate=b16(out_in))
    d = inputs_for("tiny_")
    out = O.fused_experts(d["x"], d["w13"], d["w2"], d["topk_weights"], d["topk_ids"])
    gelu = O.fused_experts(d["x"], d["w13"], d["w2"], d["topk_weights"], d["topk_ids"],
                           activation="gelu")
    np.savez_compressed(os.path.join(OUT, "tiny_M64_K128_N256_E8_k2.npz"),
                        inputs_sha256=sha(d["x"], d["w13"], d["w2"]),
                        topk_weights=d["topk_weights"].numpy(),
                        topk_ids=d["topk_ids"].numpy().astype(np.int32), out=b16(out),
                        out_gelu=b16(gelu))
    d = inputs_for("quant_")
    q13, s13 = O.block_quant_fp8(d["w13"])
    q2, s2 = O.block_quant_fp8(d["w2"])
    xq, xs = O.per_token_group_quant_fp8(d["x"])
    out8 = O.fused_experts_fp8(d["x"], q13, s13, q2, s2, d["topk_weights"], d["topk_ids"])
    i13, c13, z13 = O.quant_int4(d["w13"])
    i2, c2, z2 = O.quant_int4(d["w2"])
    out4 = O.fused_experts_w4a16(d["x"], i13, c13, z13, i2, c2, z2, d["topk_weights"], d["topk_ids"])
    np.savez_compressed(
        os.path.join(OUT, "quant_M5_K256_N128_E4_k2.npz"), inputs_sha256=sha(d["x"], d["w13"], d["w2"]),
        topk_weights=d["topk_weights"].numpy(), topk_ids=d["topk_ids"].numpy().astype(np.int32),
        fp8_weights_sha256=sha(q13.view(torch.uint8), s13, q2.view(torch.uint8), s2),
        int4_weights_sha256=sha(i13, c13.view(torch.int16), z13, i2, c2.view(torch.int16), z2),
        w13_s=s13.numpy(), w2_s=s2.numpy(), x_q=xq.view(torch.uint8).numpy(), x_s=xs.numpy(),
        out_fp8=b16(out8), out_int4=b16(out4))
    d = inputs_for("bias_")
    outb = O.fused_experts_bias(d["x"], d["w13"], d["b13"], d["w2"], d["b2"], d["topk_weights"],
                                d["topk_ids"], alpha=1.702, limit=7.0)
    np.savez_compressed(os.path.join(OUT, "bias_M6_K128_N128_E4_k2.npz"),
                        inputs_sha256=sha(d["x"], d["w13"], d["w2"], d["b13"], d["b2"]),
                        topk_weights=d["topk_weights"].numpy(),
                        topk_ids=d["topk_ids"].numpy().astype(np.int32), out=b16(outb))
    print("fixtures written to", OUT)


if __name__ == "__main__":
    main()
