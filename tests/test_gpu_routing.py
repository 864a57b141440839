"""GPU parity of the routing stages against the CPU oracle, through the C ABI:
routers (ids bit-exact, weights within fp32 ulps), moe_align (every output
bit-exact, run-to-run identical), fp8 group quant (bit-exact)."""

import numpy as np
import pytest
import torch

import flaggems_sglang
from flaggems_sglang.ops import fused_moe as F
from oracle import fused_moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ids_equal_up_to_ties(ids_gpu, ids_ref, p_ref):
    """Ids must match; a swap is tolerated only between experts whose oracle
    probabilities are exactly equal (torch.topk leaves their order open)."""
    if np.array_equal(ids_gpu, ids_ref):
        return True
    bad = np.nonzero((ids_gpu != ids_ref).any(axis=1))[0]
    for t in bad:
        a, b = set(ids_gpu[t].tolist()), set(ids_ref[t].tolist())
        vals_a = sorted(p_ref[t, list(a)].tolist())
        vals_b = sorted(p_ref[t, list(b)].tolist())
        if vals_a != vals_b:
            return False
    return True


@pytest.mark.parametrize("M,E,k", [(1, 8, 2), (64, 8, 2), (4096, 8, 2), (8192, 128, 8), (77, 1024, 32)])
def test_topk_softmax(M, E, k):
    g = torch.Generator().manual_seed(M + E + k)
    logits = torch.randn(M, E, generator=g)
    w_ref, i_ref = O.softmax_topk(logits, k)
    w, ids = flaggems_sglang.topk_softmax(logits.to(DEV), k)
    p_ref = torch.softmax(logits, -1).numpy()
    assert _ids_equal_up_to_ties(ids.cpu().numpy(), i_ref.numpy(), p_ref)
    torch.testing.assert_close(w.cpu(), w_ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("M", [1, 128, 4096])
def test_grouped_topk(M, bias):
    g = torch.Generator().manual_seed(M + 256)
    E = 256
    logits = torch.randn(M, E, generator=g)
    b = torch.randn(E, generator=g) * 0.1 if bias else None
    w_ref, i_ref = O.grouped_topk(logits, 8, 8, 4, bias=b)
    w, ids = flaggems_sglang.grouped_topk(logits.to(DEV), 8, 8, 4,
                                          correction_bias=None if b is None else b.to(DEV))
    assert np.array_equal(ids.cpu().numpy(), i_ref.numpy())
    torch.testing.assert_close(w.cpu(), w_ref, rtol=1e-5, atol=1e-6)


ALIGN_CASES = [
    # (M, E, k, expert_bias_std) -- tiny, reference small shapes, the BASELINE
    # configs' routing sizes (Qwen3 skewed, DSV3), multi-chunk sizes
    (1, 8, 2, 0.0), (7, 8, 2, 0.0), (33, 16, 4, 0.0), (64, 8, 2, 0.0), (256, 8, 2, 0.0),
    (257, 8, 2, 0.0), (1024, 128, 8, 0.5), (8192, 128, 8, 0.5), (4096, 256, 8, 0.0),
    (8192, 256, 8, 0.0), (4096, 8, 2, 0.0), (3000, 1024, 3, 2.0),
    (600, 64, 32, 0.0),  # k = 32: full 8192-slot chunks in the chunked path
    (40000, 256, 8, 0.0),  # 157 chunks: every scatter workgroup rescans 20 batches
    # one-workgroup kernel (one chunk, more than 1024 slots) and the chunked
    # path with a one-token last chunk
    (129, 32, 8, 0.0), (200, 64, 8, 1.0), (257, 16, 8, 0.0),
]


@pytest.mark.parametrize("bm", [16, 64, 128, 160, 256])
@pytest.mark.parametrize("M,E,k,bias", ALIGN_CASES)
def test_align_bit_exact(M, E, k, bias, bm):
    d = O.make_inputs(M, 8, 8, E, k, expert_bias_std=bias)
    r = O.standard_topk_to_routing(d["topk_weights"], d["topk_ids"], E)
    x = O.compute_expt_data(r["hist"], E, M * k, bm)
    s = O.moe_align_block_size(d["topk_ids"].numpy(), bm, E)
    a = F._align(d["topk_weights"].to(DEV), d["topk_ids"].to(DEV), E, bm, sglang_format=True)
    for key in ("expt_indx", "topk_indx", "gate_indx", "hist"):
        assert np.array_equal(getattr(a, key).cpu().numpy(), r[key]), key
    assert np.array_equal(a.expt_scal.cpu().numpy(), r["expt_scal"])
    assert np.array_equal(a.gate_scal.cpu().numpy(), r["gate_scal"])
    assert np.array_equal(a.offs_raw.cpu().numpy(), x["token_offs_raw"])
    assert np.array_equal(a.offs_pad.cpu().numpy(), x["token_offs_pad"])
    nt = int(a.n_tiles.item())
    assert nt == x["n_tiles"]
    tm = a.tile_map.cpu().numpy()
    assert np.array_equal(tm[: len(x["block_pid_map"])], x["block_pid_map"])
    assert np.all(tm[nt:] == -1)
    tot = int(s["num_tokens_post_padded"])
    assert int(a.num_tokens_post_padded.item()) == tot
    assert np.array_equal(a.sorted_token_ids.cpu().numpy(), s["sorted_token_ids"])
    assert np.array_equal(a.expert_ids.cpu().numpy(), s["expert_ids"])
    # determinism: a second run gives identical bits
    b = F._align(d["topk_weights"].to(DEV), d["topk_ids"].to(DEV), E, bm, sglang_format=True)
    for key in ("topk_indx", "gate_indx", "gate_scal", "sorted_token_ids", "tile_map"):
        assert torch.equal(getattr(a, key), getattr(b, key)), key


def test_align_empty_experts_and_all_one_expert():
    """Edge cases: every token on the same experts (one hot expert, the rest
    empty) and M = 0."""
    M, E, k = 300, 64, 2
    ids = torch.tensor([[5, 9]] * M, dtype=torch.int32)
    w = torch.full((M, k), 0.5)
    r = O.standard_topk_to_routing(w, ids, E)
    a = F._align(w.to(DEV), ids.to(DEV), E, 64, sglang_format=True)
    assert np.array_equal(a.topk_indx.cpu().numpy(), r["topk_indx"])
    assert np.array_equal(a.hist.cpu().numpy(), r["hist"])
    s = O.moe_align_block_size(ids.numpy(), 64, E)
    assert np.array_equal(a.sorted_token_ids.cpu().numpy(), s["sorted_token_ids"])
    z = F._align(torch.empty(0, k, device=DEV), torch.empty(0, k, dtype=torch.int32, device=DEV), E, 16, True)
    assert int(z.n_tiles.item()) == 0 and torch.all(z.offs_raw == 0)


def _e4m3_tie_rows():
    """Rows of 128-element groups whose scale is a power of two (one element
    is +-448 * 2^j), so x / scale is exact and lands on chosen points: every
    e4m3 rounding midpoint (normal and subnormal), one bf16 ulp either side of
    it, and the e4m3 values themselves, with both signs."""
    mags = []
    for e in range(-6, 9):                      # normal binades 2^-6 .. 2^8
        for f in range(8):
            v = (1 + f / 8) * 2.0 ** e
            mid = (1 + (2 * f + 1) / 16) * 2.0 ** e
            if mid <= 448:
                mags += [v, mid]
    for i in range(8):                          # subnormal codes and midpoints
        mags += [i * 2.0 ** -9, (2 * i + 1) * 2.0 ** -10]
    base = torch.tensor(mags, dtype=torch.float32)
    b16 = base.bfloat16()                       # exact: every point has <= 4 significant bits
    up = torch.nextafter(b16, torch.tensor(float("inf"), dtype=torch.bfloat16)).float()
    dn = torch.nextafter(b16, torch.tensor(0.0, dtype=torch.bfloat16)).float()
    vals = torch.cat([base, up, dn])
    vals = torch.cat([vals, -vals])             # includes -0.0 (e4m3 byte 0x80)
    n_grp = (vals.numel() + 126) // 127
    rows = []
    for j in (-12, -3, 0, 5):
        g = torch.zeros(n_grp, 128)
        flat = torch.zeros(n_grp * 127)
        flat[: vals.numel()] = vals
        g[:, 1:] = flat.view(n_grp, 127)
        g[:, 0] = 448.0 * (-1) ** torch.arange(n_grp)   # the group amax: +-448
        rows.append(g * 2.0 ** j)
    x = torch.cat(rows).view(-1, 256 if n_grp % 2 == 0 else 128)
    return x.to(torch.bfloat16)


def test_quant_fp8_ties_and_subnormals():
    """Exact rounding midpoints and e4m3 subnormals: the GPU's division and
    RNE conversion give the oracle's bytes (round half to even)."""
    x = _e4m3_tie_rows()
    assert torch.equal(x.float(), x.float().bfloat16().float())
    q_ref, s_ref = O.per_token_group_quant_fp8(x)
    assert torch.all((s_ref.log2() == s_ref.log2().round()))  # power-of-two scales
    q, s = flaggems_sglang.per_token_group_quant_fp8(x.to(DEV))
    assert torch.equal(s.cpu(), s_ref)
    assert torch.equal(q.cpu().view(torch.uint8), q_ref.view(torch.uint8))


@pytest.mark.parametrize("M,K", [(1, 128), (7, 7168), (256, 2048), (4096, 7168)])
def test_quant_fp8_bit_exact(M, K):
    g = torch.Generator().manual_seed(M + K)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    x[0, :128] = 0  # an all-zero group (eps floor)
    q_ref, s_ref = O.per_token_group_quant_fp8(x)
    q, s = flaggems_sglang.per_token_group_quant_fp8(x.to(DEV))
    assert torch.equal(s.cpu(), s_ref)
    assert torch.equal(q.cpu().view(torch.uint8), q_ref.view(torch.uint8))
