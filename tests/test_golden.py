"""Golden fixtures of the fused-MoE path (tests/golden/*.npz, written by
tests/golden/make_fixtures.py from the CPU oracle on the reference's input
recipe, tests/test_fused_moe.py:50-58).

CPU: the generator still produces the same inputs (SHA-256 of their bytes),
and the oracle still produces the stored routing, alignment and outputs bit
for bit -- a change to the oracle or to the input recipe fails here.
GPU: the HIP path, through the C ABI, against the stored outputs: routing,
alignment and quantized weights / activations bit-exact; bf16 outputs within
2e-2, fp8 / int4 within 5e-2 (the same bounds as the oracle parity tests).
"""

import hashlib
import importlib.util
import os

import numpy as np
import pytest
import torch

from oracle import fused_moe_oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
_spec = importlib.util.spec_from_file_location("make_fixtures", os.path.join(GOLD, "make_fixtures.py"))
MF = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(MF)

REF_NAMES = ["ref_M{}_K{}_N{}_E{}_k{}".format(*s) for s in MF.REF_SHAPES]


def _load(name):
    with np.load(os.path.join(GOLD, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _bf16(a):
    return torch.from_numpy(a.astype(np.uint16).view(np.int16)).view(torch.bfloat16)


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _sha(*ts):
    h = hashlib.sha256()
    for t in ts:
        h.update(t.cpu().contiguous().view(torch.uint8).numpy().tobytes())
    return np.frombuffer(h.digest(), dtype=np.uint8)


def test_fixture_files_present_and_small():
    names = sorted(f for f in os.listdir(GOLD) if f.endswith(".npz"))
    # 6 oracle fixtures (make_fixtures.py) + 1 product regression pin (make_int4_regression.py)
    assert len(names) == 7, names
    assert sum(os.path.getsize(os.path.join(GOLD, f)) for f in names) < 512 * 1024


# ------------------------------------------------------------------ CPU
@pytest.mark.parametrize("name", REF_NAMES)
def test_oracle_reproduces_reference_shape_fixture(name):
    g = _load(name)
    x, w1, w2, logits, tw, ti = MF.inputs_for(name)
    assert np.array_equal(_sha(x, w1, w2, logits), g["inputs_sha256"])
    assert np.array_equal(tw.numpy(), g["topk_weights"])
    assert np.array_equal(ti.numpy(), g["topk_ids"])
    E = w1.shape[0]
    r = O.standard_topk_to_routing(tw, ti, E)
    for key in ("topk_indx", "gate_indx", "gate_scal", "hist"):
        assert np.array_equal(np.asarray(r[key]), g[key]), key
    al = O.moe_align_block_size(ti, 16, E)
    assert np.array_equal(al["sorted_token_ids"], g["sorted_token_ids"])
    assert np.array_equal(al["expert_ids"], g["expert_ids"])
    assert int(al["num_tokens_post_padded"]) == int(g["num_tokens_post_padded"][0])
    out = O.fused_experts(x, w1.transpose(1, 2), w2.transpose(1, 2), tw, ti)
    assert np.array_equal(_bits(out), g["out"])
    out = O.fused_experts(x, w1.transpose(1, 2), w2.transpose(1, 2), tw, ti,
                          apply_router_weight_on_input=True)
    assert np.array_equal(_bits(out), g["out_input_gate"])


def test_oracle_reproduces_tiny_fixture():
    g = _load("tiny_M64_K128_N256_E8_k2")
    d = MF.inputs_for("tiny_")
    assert np.array_equal(_sha(d["x"], d["w13"], d["w2"]), g["inputs_sha256"])
    args = (d["x"], d["w13"], d["w2"], d["topk_weights"], d["topk_ids"])
    assert np.array_equal(_bits(O.fused_experts(*args)), g["out"])
    assert np.array_equal(_bits(O.fused_experts(*args, activation="gelu")), g["out_gelu"])


def test_oracle_reproduces_quant_fixture():
    g = _load("quant_M5_K256_N128_E4_k2")
    d = MF.inputs_for("quant_")
    assert np.array_equal(_sha(d["x"], d["w13"], d["w2"]), g["inputs_sha256"])
    q13, s13 = O.block_quant_fp8(d["w13"])
    q2, s2 = O.block_quant_fp8(d["w2"])
    assert np.array_equal(_sha(q13.view(torch.uint8), s13, q2.view(torch.uint8), s2),
                          g["fp8_weights_sha256"])
    xq, xs = O.per_token_group_quant_fp8(d["x"])
    assert np.array_equal(xq.view(torch.uint8).numpy(), g["x_q"])
    assert np.array_equal(xs.numpy(), g["x_s"])
    out = O.fused_experts_fp8(d["x"], q13, s13, q2, s2, d["topk_weights"], d["topk_ids"])
    assert np.array_equal(_bits(out), g["out_fp8"])
    i13, c13, z13 = O.quant_int4(d["w13"])
    i2, c2, z2 = O.quant_int4(d["w2"])
    assert np.array_equal(_sha(i13, c13.view(torch.int16), z13, i2, c2.view(torch.int16), z2),
                          g["int4_weights_sha256"])
    out = O.fused_experts_w4a16(d["x"], i13, c13, z13, i2, c2, z2, d["topk_weights"], d["topk_ids"])
    assert np.array_equal(_bits(out), g["out_int4"])


def test_oracle_reproduces_bias_fixture():
    g = _load("bias_M6_K128_N128_E4_k2")
    d = MF.inputs_for("bias_")
    assert np.array_equal(_sha(d["x"], d["w13"], d["w2"], d["b13"], d["b2"]), g["inputs_sha256"])
    out = O.fused_experts_bias(d["x"], d["w13"], d["b13"], d["w2"], d["b2"], d["topk_weights"],
                               d["topk_ids"], alpha=1.702, limit=7.0)
    assert np.array_equal(_bits(out), g["out"])


# ------------------------------------------------------------------ GPU
DEV = "cuda"


def _close(out, ref, tol):
    """Same bound as the oracle parity tests: elementwise within
    tol * (rms(ref) + |ref|) and global relative error below tol / 4."""
    out = out.float().cpu()
    ref = ref.float()
    scale = max(float(ref.pow(2).mean().sqrt()), 1e-3)
    torch.testing.assert_close(out, ref, atol=tol * scale, rtol=tol)
    rel = float((out - ref).norm() / ref.norm().clamp_min(1e-30))
    assert rel < tol / 4, f"global relative error {rel:.3e}"


@pytest.mark.gpu
@pytest.mark.parametrize("name", REF_NAMES)
def test_gpu_reference_shape_fixture(name):
    import flaggems_sglang
    from flaggems_sglang.ops import fused_moe as F

    g = _load(name)
    x, w1, w2, logits, _, _ = MF.inputs_for(name)
    E, k = w1.shape[0], g["topk_ids"].shape[1]
    tw, ti = F.topk_softmax(logits.to(DEV), k)
    assert np.array_equal(ti.int().cpu().numpy(), g["topk_ids"])
    torch.testing.assert_close(tw.cpu(), torch.from_numpy(g["topk_weights"]), atol=1e-6, rtol=1e-6)
    tw = torch.from_numpy(g["topk_weights"]).to(DEV)
    ti = torch.from_numpy(g["topk_ids"]).to(DEV)
    a = F._align(tw, ti, E, 16, sglang_format=True)
    for key in ("topk_indx", "gate_indx", "gate_scal", "hist", "sorted_token_ids", "expert_ids"):
        assert np.array_equal(getattr(a, key).cpu().numpy(), g[key]), key
    assert int(a.num_tokens_post_padded.item()) == int(g["num_tokens_post_padded"][0])
    rd, gi, si = F._standard_topk_to_triton_kernels(tw, ti, E)
    for on_input, key in ((False, "out"), (True, "out_input_gate")):
        out = flaggems_sglang.triton_kernel_fused_experts(
            x.to(DEV), w1.to(DEV), w2.to(DEV), rd, gi, si, apply_router_weight_on_input=on_input)
        _close(out, _bf16(g[key]), 2e-2)


@pytest.mark.gpu
@pytest.mark.parametrize("path", [0, 1, 2])
def test_gpu_tiny_fixture(path):
    import flaggems_sglang

    g = _load("tiny_M64_K128_N256_E8_k2")
    d = MF.inputs_for("tiny_")
    args = [d["x"].to(DEV), d["w13"].to(DEV), d["w2"].to(DEV),
            torch.from_numpy(g["topk_weights"]).to(DEV), torch.from_numpy(g["topk_ids"]).to(DEV)]
    _close(flaggems_sglang.fused_experts(*args, path=path), _bf16(g["out"]), 2e-2)
    _close(flaggems_sglang.fused_experts(*args, activation="gelu", path=path), _bf16(g["out_gelu"]), 2e-2)


@pytest.mark.gpu
def test_gpu_quant_fixture():
    import flaggems_sglang
    from flaggems_sglang import quant as Q
    from flaggems_sglang.ops import fused_moe as F

    g = _load("quant_M5_K256_N128_E4_k2")
    d = MF.inputs_for("quant_")
    tw = torch.from_numpy(g["topk_weights"]).to(DEV)
    ti = torch.from_numpy(g["topk_ids"]).to(DEV)
    x = d["x"].to(DEV)
    q13, s13 = Q.quantize_fp8_block(d["w13"].to(DEV))
    q2, s2 = Q.quantize_fp8_block(d["w2"].to(DEV))
    assert np.array_equal(_sha(q13.view(torch.uint8), s13, q2.view(torch.uint8), s2),
                          g["fp8_weights_sha256"])
    xq, xs = F.per_token_group_quant_fp8(x, 128)
    assert np.array_equal(xq.view(torch.uint8).cpu().numpy(), g["x_q"])
    assert np.array_equal(xs.cpu().numpy(), g["x_s"])
    for path in (1, 2):
        out = flaggems_sglang.fused_experts(x, q13, q2, tw, ti, use_fp8_w8a8=True, w1_scale=s13,
                                            w2_scale=s2, block_shape=[128, 128], path=path)
        _close(out, _bf16(g["out_fp8"]), 5e-2)
    i13, c13, z13 = Q.quantize_int4_group(d["w13"].to(DEV))
    i2, c2, z2 = Q.quantize_int4_group(d["w2"].to(DEV))
    assert np.array_equal(_sha(i13, c13.view(torch.int16), z13, i2, c2.view(torch.int16), z2),
                          g["int4_weights_sha256"])
    out = flaggems_sglang.fused_experts(x, i13, i2, tw, ti, use_int4_w4a16=True, w1_scale=c13,
                                        w2_scale=c2, w1_zp=z13, w2_zp=z2)
    _close(out, _bf16(g["out_int4"]), 5e-2)


@pytest.mark.gpu
def test_gpu_bias_fixture():
    import flaggems_sglang
    from flaggems_sglang.ops import fused_moe as F

    g = _load("bias_M6_K128_N128_E4_k2")
    d = MF.inputs_for("bias_")
    tw = torch.from_numpy(g["topk_weights"]).to(DEV)
    ti = torch.from_numpy(g["topk_ids"]).to(DEV)
    rd, gi, si = F._standard_topk_to_triton_kernels(tw, ti, 4)
    out = flaggems_sglang.triton_kernel_fused_experts_with_bias(
        d["x"].to(DEV), d["w13"].transpose(1, 2).to(DEV), None, d["b13"].to(DEV),
        d["w2"].transpose(1, 2).to(DEV), None, d["b2"].to(DEV), rd, gi, si,
        gemm1_alpha=1.702, gemm1_clamp_limit=7.0)
    _close(out, _bf16(g["out"]), 2e-2)
