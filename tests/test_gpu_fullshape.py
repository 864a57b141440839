"""Full BASELINE shapes on the GPU, through the C ABI.

Where the CPU oracle finishes in seconds the whole output is compared
(DeepSeek-V3 fp8 at E=256 for M = 1 and 128 -- the oracle dequantizes only
the experts the tokens hit; Mixtral bf16 at M = 1 and 256).  At the large
prefill sizes (DeepSeek-V3 fp8 M=4096 and 8192, Qwen3 bf16 M=8192) the checks are the
size-independent ones: bit identity across runs, exact token-permutation
equivariance, and an 8-token spot check against the oracle.

Weights are generated on the GPU in expert chunks (the DeepSeek-V3 layer is
11.3 GB in fp8); only the experts the oracle needs are copied to the host.
Tolerances: bf16 2e-2, fp8 5e-2 against the dequantize-then-compute oracle.
"""

import pytest
import torch

import flaggems_sglang
from flaggems_sglang import quant as Q
from oracle import fused_moe_oracle as O

from test_gpu_fused_moe import _close, _close_literal

pytestmark = pytest.mark.gpu
DEV = "cuda"


class _HostExperts:
    """Indexable view of a device weight tensor [E, ...]: item e is copied
    to the host on demand, so the oracle touches only the experts it uses."""

    def __init__(self, t):
        self.t = t
        self.shape = t.shape

    def __getitem__(self, e):
        return self.t[e].cpu()


def _gpu_weights(E, R, C, seed, std=0.02, chunk=16, fp8=False):
    """[E, R, C] ~ N(0, std) bf16 (or its 128x128 block-fp8 quantization),
    generated chunk by chunk on the device."""
    gen = torch.Generator(device=DEV).manual_seed(seed)
    if fp8:
        q = torch.empty(E, R, C, dtype=torch.float8_e4m3fn, device=DEV)
        s = torch.empty(E, R // 128, C // 128, dtype=torch.float32, device=DEV)
    else:
        q = torch.empty(E, R, C, dtype=torch.bfloat16, device=DEV)
    for e0 in range(0, E, chunk):
        n = min(chunk, E - e0)
        w = (torch.randn(n, R, C, device=DEV, generator=gen) * std).to(torch.bfloat16)
        if fp8:
            q[e0:e0 + n], s[e0:e0 + n] = Q.quantize_fp8_block(w)
        else:
            q[e0:e0 + n] = w
        del w
    return (q, s) if fp8 else q


# ------------------------------------------------------------ DeepSeek-V3 fp8
K3, N3, E3, k3 = 7168, 2048, 256, 8


@pytest.fixture(scope="module")
def dsv3_layer():
    q1, s1 = _gpu_weights(E3, 2 * N3, K3, seed=31, fp8=True)
    q2, s2 = _gpu_weights(E3, K3, N3, seed=32, fp8=True)
    yield q1, s1, q2, s2
    del q1, s1, q2, s2
    torch.cuda.empty_cache()


def _dsv3_routing(M, seed):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(M, K3, device=DEV, generator=gen).to(torch.bfloat16)
    logits = torch.randn(M, E3, device=DEV, generator=gen)
    tw, ti = flaggems_sglang.grouped_topk(logits, k3, num_expert_group=8, topk_group=4)
    return x, tw, ti


def _dsv3_call(layer, x, tw, ti):
    q1, s1, q2, s2 = layer
    return flaggems_sglang.fused_experts(x, q1, q2, tw, ti, use_fp8_w8a8=True, w1_scale=s1,
                                         w2_scale=s2, block_shape=[128, 128])


def _dsv3_oracle(layer, x, tw, ti):
    q1, s1, q2, s2 = layer
    return O.fused_experts_fp8(x.cpu(), _HostExperts(q1), _HostExperts(s1), _HostExperts(q2),
                               _HostExperts(s2), tw.cpu(), ti.cpu())


@pytest.mark.parametrize("M", [1, 128])
def test_dsv3_fp8_full_experts(dsv3_layer, M):
    """E=256, grouped routing (8 groups, top-4 groups, top-8 experts), full
    K / N: the whole output against the oracle."""
    x, tw, ti = _dsv3_routing(M, seed=100 + M)
    out = _dsv3_call(dsv3_layer, x, tw, ti)
    ref = _dsv3_oracle(dsv3_layer, x, tw, ti)
    _close(out, ref, 5e-2)
    _close_literal(out, ref, 5e-2)


def _permutation_checks(call, oracle, x, tw, ti, tol, seed):
    a = call(x, tw, ti)
    b = call(x, tw, ti)
    assert torch.equal(a, b), "not bit-identical across runs"
    M = x.shape[0]
    gen = torch.Generator(device=DEV).manual_seed(seed)
    perm = torch.randperm(M, device=DEV, generator=gen)
    c = call(x[perm], tw[perm], ti[perm])
    assert torch.equal(c, a[perm]), "token permutation does not permute the output exactly"
    sel = perm[:8]
    _close(a[sel], oracle(x[sel], tw[sel], ti[sel]), tol)


@pytest.mark.parametrize("M", [4096, 8192])
def test_dsv3_fp8_prefill_permutation_and_determinism(dsv3_layer, M):
    x, tw, ti = _dsv3_routing(M, seed=M)
    _permutation_checks(lambda *a: _dsv3_call(dsv3_layer, *a),
                        lambda *a: _dsv3_oracle(dsv3_layer, *a), x, tw, ti, 5e-2, seed=9)


# ------------------------------------------------------------ Qwen3 bf16 M=8192
def test_qwen3_bf16_m8192_permutation_and_determinism():
    M, K, N, E, k = 8192, 2048, 768, 128, 8
    w13 = _gpu_weights(E, 2 * N, K, seed=41)
    w2 = _gpu_weights(E, K, N, seed=42)
    gen = torch.Generator(device=DEV).manual_seed(43)
    x = torch.randn(M, K, device=DEV, generator=gen).to(torch.bfloat16)
    # per-expert bias N(0, 0.5) on the logits skews the routing
    logits = torch.randn(M, E, device=DEV, generator=gen) + \
        torch.randn(E, device=DEV, generator=gen)[None, :] * 0.5
    tw, ti = flaggems_sglang.topk_softmax(logits, k)

    def oracle(xs, ws, ids):
        return O.fused_experts(xs.cpu(), _HostExperts(w13), _HostExperts(w2), ws.cpu(), ids.cpu())

    _permutation_checks(lambda *a: flaggems_sglang.fused_experts(a[0], w13, w2, a[1], a[2]),
                        oracle, x, tw, ti, 2e-2, seed=10)


# ------------------------------------------------------------ Mixtral bf16
@pytest.mark.parametrize("M", [1, 256])
def test_mixtral_bf16_full_shape(M):
    """Mixtral-8x7B shape (E=8, top-2, K=4096, N=14336) at M = 1 (decode
    kernels, in-workgroup routing) and M = 256 (prefill kernels)."""
    K, N, E, k = 4096, 14336, 8, 2
    w13 = _gpu_weights(E, 2 * N, K, seed=51, chunk=2)
    w2 = _gpu_weights(E, K, N, seed=52, chunk=2)
    gen = torch.Generator(device=DEV).manual_seed(53 + M)
    x = torch.randn(M, K, device=DEV, generator=gen).to(torch.bfloat16)
    tw, ti = flaggems_sglang.topk_softmax(torch.randn(M, E, device=DEV, generator=gen), k)
    out = flaggems_sglang.fused_experts(x, w13, w2, tw, ti)
    ref = O.fused_experts(x.cpu(), _HostExperts(w13), _HostExperts(w2), tw.cpu(), ti.cpu())
    _close(out, ref, 2e-2)
    _close_literal(out, ref, 2e-2)
