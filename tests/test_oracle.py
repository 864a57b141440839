"""Pins the CPU oracle (``oracle/fused_moe_oracle.py``) before anything is
checked against it.

The reference holds no golden vectors for this path (its fused-MoE test
compares against SGLang live on a GPU, ``tests/test_fused_moe.py:93-96``), so
each oracle function is pinned by something independent of its own formula:
brute-force loops on small inputs, closed forms that reduce to a library or
textbook routine, and invariants chosen so that a dropped term, a wrong index
or a transposed operand fails.
"""

import math

import numpy as np
import pytest
import scipy.special
import torch

from oracle import fused_moe_oracle as O


# ----------------------------------------------------------------- routing
def _bf_softmax_topk(logits, k):
    out_w, out_i = [], []
    for row in logits.tolist():
        m = max(row)
        ex = [math.exp(v - m) for v in row]
        s = sum(ex)
        p = [v / s for v in ex]
        order = sorted(range(len(p)), key=lambda i: -p[i])[:k]
        w = [p[i] for i in order]
        ws = sum(w)
        out_w.append([v / ws for v in w])
        out_i.append(order)
    return np.array(out_w), np.array(out_i)


@pytest.mark.parametrize("M,E,k", [(5, 8, 2), (9, 16, 4), (3, 128, 8)])
def test_softmax_topk_bruteforce(M, E, k):
    g = torch.Generator().manual_seed(M * E + k)
    logits = torch.randn(M, E, generator=g)
    w, ids = O.softmax_topk(logits, k)
    bw, bi = _bf_softmax_topk(logits.double(), k)
    assert np.array_equal(ids.numpy(), bi)
    np.testing.assert_allclose(w.numpy(), bw, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(w.sum(-1).numpy(), 1.0, rtol=1e-6)


def _bf_grouped(logits, k, n_group, topk_group, bias):
    M, E = logits.shape
    gsz = E // n_group
    W, I = [], []
    for t in range(M):
        s = [1.0 / (1.0 + math.exp(-float(v))) for v in logits[t]]
        sel = [s[e] + (float(bias[e]) if bias is not None else 0.0) for e in range(E)]
        gscore = []
        for g in range(n_group):
            vals = sorted(sel[g * gsz:(g + 1) * gsz], reverse=True)
            gscore.append(vals[0] + vals[1])
        keep = sorted(range(n_group), key=lambda g: -gscore[g])[:topk_group]
        cand = [e for e in range(E) if e // gsz in keep]
        chosen = sorted(cand, key=lambda e: -sel[e])[:k]
        w = [s[e] for e in chosen]
        tot = sum(w)
        W.append([v / tot for v in w])
        I.append(chosen)
    return np.array(W), np.array(I)


@pytest.mark.parametrize("bias", [False, True])
def test_grouped_topk_bruteforce(bias):
    g = torch.Generator().manual_seed(7)
    M, E = 6, 64
    logits = torch.randn(M, E, generator=g)
    b = torch.randn(E, generator=g) * 0.5 if bias else None
    w, ids = O.grouped_topk(logits, 8, 8, 4, bias=b)
    bw, bi = _bf_grouped(logits.double(), 8, 8, 4, b)
    assert np.array_equal(ids.numpy(), bi)
    np.testing.assert_allclose(w.numpy(), bw, rtol=1e-5)
    # every chosen expert lies in at most topk_group groups
    assert all(len(set((ids[t] // 8).tolist())) <= 4 for t in range(M))


# ---------------------------------------------------- routing conversion
def _bf_routing(w, ids, E):
    M, k = ids.shape
    rows = []
    for t in range(M):
        pairs = sorted(zip(ids[t].tolist(), w[t].tolist()))
        rows.append(pairs)
    flat = [p for r in rows for p in r]
    buckets = [[] for _ in range(E)]
    for f, (e, wt) in enumerate(flat):
        buckets[e].append(f)
    topk_indx = [f for b in buckets for f in b]
    gate_indx = [0] * len(flat)
    for s, f in enumerate(topk_indx):
        gate_indx[f] = s
    return dict(
        expt_indx=[e for e, _ in flat],
        topk_indx=topk_indx,
        gate_indx=gate_indx,
        gate_scal=[flat[f][1] for f in topk_indx],
        hist=[len(b) for b in buckets],
    )


@pytest.mark.parametrize("M,E,k", [(1, 8, 2), (7, 8, 2), (33, 16, 4), (50, 128, 8), (3, 256, 8)])
def test_routing_conversion_bruteforce(M, E, k):
    d = O.make_inputs(M, 16, 16, E, k)
    r = O.standard_topk_to_routing(d["topk_weights"], d["topk_ids"], E)
    b = _bf_routing(d["topk_weights"].numpy(), d["topk_ids"].numpy(), E)
    for key in ("expt_indx", "topk_indx", "gate_indx", "hist"):
        assert np.array_equal(r[key], np.array(b[key])), key
    np.testing.assert_array_equal(r["gate_scal"], np.array(b["gate_scal"], dtype=np.float32))
    # invariants: permutation, inverse, stable order, bincount
    n = M * k
    assert np.array_equal(np.sort(r["topk_indx"]), np.arange(n))
    assert np.array_equal(r["gate_indx"][r["topk_indx"]], np.arange(n))
    assert np.all(np.diff(r["expt_indx"][r["topk_indx"]]) >= 0)
    assert r["hist"].sum() == n


def _bf_expt_data(hist, E, n_gates, bm):
    offs_raw = [0]
    for h in hist:
        offs_raw.append(offs_raw[-1] + int(h))
    offs_pad = [0]
    for h in hist:
        offs_pad.append(offs_pad[-1] + (int(h) + bm - 1) // bm)
    # upper bound on used tiles: one partial tile per non-empty expert
    L = O.max_n_tiles(E, n_gates)
    m = [-1] * L
    for e in range(E):
        for b in range((int(hist[e]) + bm - 1) // bm):
            m[offs_pad[e] + b] = (b << 16) + e
    return offs_raw, offs_pad, m


@pytest.mark.parametrize("bm", [16, 32, 64, 128])
@pytest.mark.parametrize("M,E,k,bias", [(1, 8, 2, 0), (64, 8, 2, 0), (33, 16, 4, 0), (300, 128, 8, 0.5)])
def test_expt_data_bruteforce(bm, M, E, k, bias):
    d = O.make_inputs(M, 16, 16, E, k, expert_bias_std=bias)
    r = O.standard_topk_to_routing(d["topk_weights"], d["topk_ids"], E)
    x = O.compute_expt_data(r["hist"], E, M * k, bm)
    a, b, m = _bf_expt_data(r["hist"], E, M * k, bm)
    assert x["token_offs_raw"].tolist() == a
    assert x["token_offs_pad"].tolist() == b
    assert x["block_pid_map"].tolist() == m
    # the tile map length always covers the used tiles
    assert x["n_tiles"] <= len(m)


def _bf_align(ids, bm, E):
    M, k = ids.shape
    flat = ids.reshape(-1).tolist()
    out, eids = [], []
    for e in range(E):
        seg = [i for i, v in enumerate(flat) if v == e]
        if not seg:
            continue
        pad = (len(seg) + bm - 1) // bm * bm
        out += seg + [M * k] * (pad - len(seg))
        eids += [e] * (pad // bm)
    return out, eids


@pytest.mark.parametrize("bm", [16, 64])
@pytest.mark.parametrize("M,E,k", [(1, 8, 2), (37, 16, 4), (200, 128, 8)])
def test_moe_align_bruteforce(bm, M, E, k):
    d = O.make_inputs(M, 16, 16, E, k, expert_bias_std=0.5)
    ids = d["topk_ids"].numpy()
    a = O.moe_align_block_size(ids, bm, E)
    out, eids = _bf_align(ids, bm, E)
    tot = int(a["num_tokens_post_padded"])
    assert tot == len(out)
    assert a["sorted_token_ids"][:tot].tolist() == out
    assert np.all(a["sorted_token_ids"][tot:] == M * k)
    assert a["expert_ids"][: tot // bm].tolist() == eids
    assert np.all(a["expert_ids"][tot // bm:] == -1)


# ------------------------------------------------------------- activation
def test_silu_and_mul_closed_form():
    g = torch.Generator().manual_seed(0)
    inter = (torch.randn(17, 2 * 96, generator=g) * 4).to(torch.bfloat16)
    got = O.silu_and_mul(inter)
    gate = inter[:, :96].double().numpy()
    up = inter[:, 96:].double().numpy()
    want = gate * scipy.special.expit(gate) * up
    np.testing.assert_allclose(got.numpy(), want, rtol=2e-6, atol=1e-6)
    # special values: silu(0) = 0, silu(x) -> x for large x, gate/up not swapped
    t = torch.tensor([[0.0, 20.0, 1.0, 1.0, 3.0, 0.0]], dtype=torch.bfloat16)
    r = O.silu_and_mul(t)
    assert r[0, 0] == 0 and abs(float(r[0, 1]) - 20.0 * 3.0) < 1e-3 and r[0, 2] == 0


# ---------------------------------------------------------- fused experts
@pytest.mark.parametrize("shape", [(1, 128, 256, 8, 2), (7, 128, 256, 8, 2), (33, 256, 512, 16, 4)])
def test_fused_experts_vs_bruteforce(shape):
    """The reference's FUSED_MOE_SHAPES_SMALL (tests/accuracy_utils.py:100-104)."""
    M, K, N, E, k = shape
    d = O.make_inputs(M, K, N, E, k, wscale=0.1)
    got = O.fused_experts(d["x"], d["w13"], d["w2"], d["topk_weights"], d["topk_ids"])
    bf = O.fused_experts_bruteforce(d["x"], d["w13"], d["w2"], d["topk_weights"], d["topk_ids"])
    torch.testing.assert_close(got.double(), bf, rtol=2e-2, atol=2e-2 * bf.abs().max().item())


def test_fused_experts_dense_special_case():
    """E=1, k=1, weight 1: the MoE reduces to a dense SwiGLU MLP."""
    g = torch.Generator().manual_seed(3)
    M, K, N = 9, 64, 32
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w13 = (torch.randn(1, 2 * N, K, generator=g) * 0.1).to(torch.bfloat16)
    w2 = (torch.randn(1, K, N, generator=g) * 0.1).to(torch.bfloat16)
    w = torch.ones(M, 1)
    ids = torch.zeros(M, 1, dtype=torch.int32)
    got = O.fused_experts(x, w13, w2, w, ids)
    xf = x.double()
    h = torch.nn.functional.silu(xf @ w13[0, :N].double().t()) * (xf @ w13[0, N:].double().t())
    want = h @ w2[0].double().t()
    torch.testing.assert_close(got.double(), want, rtol=2e-2, atol=2e-2)


def test_fused_experts_router_weight_on_input():
    """With weights on the input side, linearity fails only through silu: for
    weights == 1 both placements agree exactly."""
    d = O.make_inputs(8, 128, 256, 8, 2, wscale=0.1)
    ones = torch.ones_like(d["topk_weights"])
    a = O.fused_experts(d["x"], d["w13"], d["w2"], ones, d["topk_ids"])
    b = O.fused_experts(d["x"], d["w13"], d["w2"], ones, d["topk_ids"], apply_router_weight_on_input=True)
    assert torch.equal(a, b)
    c = O.fused_experts(d["x"], d["w13"], d["w2"], d["topk_weights"], d["topk_ids"])
    assert not torch.equal(a, c)


def test_routed_scaling_factor():
    d = O.make_inputs(4, 128, 256, 8, 2, wscale=0.1)
    a = O.fused_experts(d["x"], d["w13"], d["w2"], d["topk_weights"], d["topk_ids"])
    b = O.fused_experts(d["x"], d["w13"], d["w2"], d["topk_weights"], d["topk_ids"], routed_scaling_factor=2.0)
    torch.testing.assert_close(b.float(), a.float() * 2.0, rtol=1e-2, atol=1e-3)


# -------------------------------------------------------------------- fp8
def test_fp8_group_quant_known_answers():
    # a group holding exact powers of two: amax 4 -> scale 4/448, every
    # element lands on an exactly representable e4m3 value
    x = torch.zeros(1, 128)
    x[0, :4] = torch.tensor([4.0, -2.0, 1.0, 0.5])
    q, s = O.per_token_group_quant_fp8(x)
    assert s.shape == (1, 1) and abs(float(s) - 4.0 / 448.0) < 1e-9
    assert float(q[0, 0].float()) == 448.0
    deq = O.dequant_token_group(q, s)
    np.testing.assert_allclose(deq[0, :4].numpy(), [4.0, -2.0, 1.0, 0.5], rtol=1e-6)
    # all-zero group: eps floor, no NaN
    q0, s0 = O.per_token_group_quant_fp8(torch.zeros(2, 256))
    assert torch.all(q0.float() == 0) and torch.all(s0 > 0)


def test_fp8_group_quant_error_bound():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(64, 512, generator=g).to(torch.bfloat16)
    q, s = O.per_token_group_quant_fp8(x)
    deq = O.dequant_token_group(q, s)
    xf = x.float()
    # e4m3 has 3 mantissa bits: relative error <= 2^-4 for normals; the
    # group's amax element maps to exactly +-448
    err = (deq - xf).abs()
    bound = xf.abs() * 2.0 ** -4 + s.repeat_interleave(128, 1) * 2.0 ** -9 * 2
    assert torch.all(err <= bound + 1e-12)
    amax_pos = xf.view(64, 4, 128).abs().argmax(-1)
    qa = q.float().view(64, 4, 128).gather(-1, amax_pos[..., None]).abs()
    assert torch.all(qa == 448.0)


def test_fp8_block_quant_roundtrip():
    g = torch.Generator().manual_seed(2)
    w = (torch.randn(2, 256, 384, generator=g) * 0.02).to(torch.bfloat16)
    q, s = O.block_quant_fp8(w)
    assert s.shape == (2, 2, 3)
    for e in range(2):
        d = O.dequant_block(q[e], s[e])
        sb = s[e].repeat_interleave(128, 0).repeat_interleave(128, 1)
        # normals: relative 2^-4; subnormals (below 2^-6 * scale): half a
        # spacing of 2^-9 * scale
        bound = w[e].float().abs() * 2 ** -4 + sb * 2 ** -10
        assert torch.all((d - w[e].float()).abs() <= bound * (1 + 1e-6))
        # a scale belongs to its own block: perturbing one block's scale moves
        # only that block
        s2 = s[e].clone()
        s2[1, 2] *= 2
        d2 = O.dequant_block(q[e], s2)
        diff = (d2 != d)
        assert diff[128:, 256:].any() and not diff[:128].any() and not diff[:, :256].any()


def test_fused_experts_fp8_close_to_bf16():
    d = O.make_inputs(16, 256, 256, 8, 2, wscale=0.02)
    q1, s1 = O.block_quant_fp8(d["w13"])
    q2, s2 = O.block_quant_fp8(d["w2"])
    got = O.fused_experts_fp8(d["x"], q1, s1, q2, s2, d["topk_weights"], d["topk_ids"])
    ref = O.fused_experts(d["x"], d["w13"], d["w2"], d["topk_weights"], d["topk_ids"])
    err = (got.float() - ref.float()).abs().max() / ref.float().abs().max()
    assert err < 0.1


# ------------------------------------------------------------------- int4
def test_int4_pack_roundtrip():
    g = torch.Generator().manual_seed(4)
    q = torch.randint(0, 16, (3, 5, 37), generator=g, dtype=torch.uint8)
    p = O.pack_u4(q)
    assert p.shape == (3, 5, 19)
    assert torch.equal(O.unpack_u4(p, 37), q)
    # nibble order: element 0 in the low nibble
    assert O.pack_u4(torch.tensor([[1, 2]], dtype=torch.uint8)).item() == 0x21


def test_int4_dequant_closed_form():
    # a group spanning [-1, 0.875] in steps of 0.125: scale 0.125 exactly,
    # zero 8, so (q - 8) * 0.125 reproduces every input
    vals = torch.arange(-8, 8, dtype=torch.float32) * 0.125
    w = vals.repeat(8).view(1, 1, 128)
    qw, sc, z = O.quant_int4(w)
    assert float(sc) == 0.125 and int(O.unpack_u4(z, 1)) == 8
    assert sc.shape == (1, 1, 1) and z.shape == (1, 1, 1)
    torch.testing.assert_close(O.dequant_int4(qw[0], sc[0], z[0]), w[0], rtol=0, atol=0)


def test_int4_quant_error_bound():
    g = torch.Generator().manual_seed(5)
    w = torch.randn(2, 64, 512, generator=g) * 0.02
    qw, sc, z = O.quant_int4(w)
    for e in range(2):
        d = O.dequant_int4(qw[e], sc[e], z[e])
        s = sc[e].float().t().repeat_interleave(128, 1)
        assert torch.all((d - w[e]).abs() <= s * 0.5 + s * 2e-3)


# ------------------------------------------------------------ activations / bias path
def test_gelu_and_mul_library_and_known_values():
    g = torch.linspace(-6, 6, 241)
    u = torch.linspace(-2, 3, 241)
    got = O.gelu_and_mul(torch.cat([g, u]).view(1, -1))[0]
    ref = torch.nn.functional.gelu(g.double(), approximate="none") * u.double()
    assert torch.allclose(got.double(), ref, atol=1e-6, rtol=1e-6)
    one = O.gelu_and_mul(torch.tensor([[1.0, 1.0]]))[0, 0].item()
    assert abs(one - 0.8413447460685429) < 1e-6          # Phi(1)
    x = torch.linspace(-4, 4, 81)
    pos = O.gelu_and_mul(torch.cat([x, torch.ones(81)]).view(1, -1))[0]
    neg = O.gelu_and_mul(torch.cat([-x, torch.ones(81)]).view(1, -1))[0]
    assert torch.allclose(pos - neg, x, atol=1e-6)        # gelu(x) - gelu(-x) = x


def test_swiglu_reduces_to_silu_and_clamps():
    g = torch.linspace(-8, 8, 161)
    inter = torch.zeros(1, 2 * g.numel())
    inter[0, 0::2] = g                                    # gate even, linear odd (= 0)
    got = O.swiglu(inter, alpha=1.0, limit=None)[0]
    assert torch.allclose(got, torch.nn.functional.silu(g), atol=1e-6)
    a, lim = 1.702, 7.0
    inter = torch.tensor([[10.0, 10.0, 10.0, -10.0, -3.0, 2.0]])
    got = O.swiglu(inter, alpha=a, limit=lim)[0]
    sig = lambda z: 1.0 / (1.0 + math.exp(-z))           # noqa: E731
    want = [lim * sig(a * lim) * (lim + 1), lim * sig(a * lim) * (-lim + 1), -3 * sig(-3 * a) * 3]
    assert torch.allclose(got.double(), torch.tensor(want, dtype=torch.float64), rtol=1e-6)


def test_fused_experts_gelu_dense_geglu():
    """E=1, k=1 with weight 1: the MoE is a dense GeGLU MLP with the same
    rounding points, written with torch's gelu (library routine)."""
    d = O.make_inputs(9, 64, 32, 1, 1, wscale=0.2)
    tw = torch.ones(9, 1)
    got = O.fused_experts(d["x"], d["w13"], d["w2"], tw, d["topk_ids"], activation="gelu")
    w13, w2 = d["w13"][0].float(), d["w2"][0].float()
    inter = (d["x"].float() @ w13.t()).to(torch.bfloat16).float()
    g, u = inter[:, :32], inter[:, 32:]
    act = (torch.nn.functional.gelu(g) * u).to(torch.bfloat16).float()
    ref = (act @ w2.t()).to(torch.bfloat16)
    assert torch.allclose(got.float(), ref.float(), atol=2e-2, rtol=1e-2)


def test_fused_experts_bias_matches_bruteforce():
    d = O.make_inputs(13, 128, 64, 6, 2, wscale=0.1)
    gen = torch.Generator().manual_seed(5)
    b13 = torch.randn(6, 128, generator=gen) * 0.2
    b2 = torch.randn(6, 128, generator=gen) * 0.2
    for alpha, limit in ((1.0, None), (1.702, 0.5)):
        got = O.fused_experts_bias(d["x"], d["w13"], b13, d["w2"], b2, d["topk_weights"],
                                   d["topk_ids"], alpha=alpha, limit=limit)
        ref = O.fused_experts_bias_bruteforce(d["x"], d["w13"], b13, d["w2"], b2, d["topk_weights"],
                                              d["topk_ids"], alpha=alpha, limit=limit)
        err = (got.double() - ref).abs().max().item()
        assert err < 2e-2 * max(1.0, ref.abs().max().item()), err


def test_fused_experts_bias_zero_weights_closed_form():
    """Zero weights: every slot's output is its expert's b2, so the MoE
    returns sum_j w_j * b2[e_j]."""
    d = O.make_inputs(7, 128, 64, 5, 3, wscale=0.1)
    gen = torch.Generator().manual_seed(9)
    b13 = torch.randn(5, 128, generator=gen)
    b2 = torch.randn(5, 128, generator=gen)
    z13 = torch.zeros_like(d["w13"])
    z2 = torch.zeros_like(d["w2"])
    got = O.fused_experts_bias(d["x"], z13, b13, z2, b2, d["topk_weights"], d["topk_ids"])
    want = (d["topk_weights"][..., None] * b2[d["topk_ids"].long()]).sum(1)
    assert torch.allclose(got.float(), want, atol=1e-2, rtol=1e-2)


def test_ep_localize_identity_and_rank_sum():
    d = O.make_inputs(11, 128, 64, 8, 3, wscale=0.1)
    full = O.fused_experts(d["x"], d["w13"], d["w2"], d["topk_weights"], d["topk_ids"])
    tw, ti = O.ep_localize(d["topk_weights"], d["topk_ids"], torch.arange(8))
    same = O.fused_experts(d["x"], d["w13"], d["w2"], tw, ti)
    assert torch.equal(full, same)
    # two ranks owning experts {0..3} and {4..7}: partial outputs sum to the
    # full one (up to the bf16 rounding of each partial)
    parts = []
    for r in range(2):
        emap = torch.full((8,), -1)
        emap[4 * r:4 * r + 4] = torch.arange(4)
        tw, ti = O.ep_localize(d["topk_weights"], d["topk_ids"], emap)
        parts.append(O.fused_experts(d["x"], d["w13"][4 * r:4 * r + 4], d["w2"][4 * r:4 * r + 4], tw, ti))
    s = parts[0].float() + parts[1].float()
    assert torch.allclose(s, full.float(), atol=2e-2 * full.float().abs().max().item(), rtol=2e-2)
