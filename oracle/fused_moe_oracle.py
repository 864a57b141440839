"""CPU oracle for the fused-MoE hot path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker / the timed CPU baseline.  The product path (``flaggems_sglang``) never
imports it and fails loudly when its HIP library is missing.

This is a restatement, in numpy / torch-on-CPU, of what FlagGems-sglang's fused
MoE computes.  Every function cites the reference file:line it follows
(paths relative to the reference root, ``src/flaggems_sglang/...``).  The
reference itself cannot run here: ``ops/fused_moe.py:16`` imports the
third-party ``triton_kernels.matmul_ogs`` (OpenAI Triton ``python/triton_kernels``,
version unpinned by the reference's ``pyproject.toml``), which is absent, and
the package's import-time device probing needs an NVIDIA GPU.

Pinning status of each function (checks live in ``tests/test_oracle.py``):

=============================  ===============================================
function                       pinned by
=============================  ===============================================
softmax_topk                   brute-force per-row sort on small inputs;
                               ``torch.topk`` semantics (library routine)
grouped_topk                   brute-force per-row loops (python) on small
                               inputs.  The routine itself is SGLang's
                               ``biased_grouped_topk`` (external, not in the
                               reference): parity to SGLang is *unpinned*.
standard_topk_to_routing       brute-force counting sort written as loops;
                               invariants (permutation, inverse, bincount)
compute_expt_data              brute-force loops + invariants.  The encoding
                               ``(block << 16) | expert`` and ``max_n_tiles``
                               follow upstream triton_kernels from its
                               published source, which is not present here:
                               *parity to triton_kernels unpinned*.
moe_align_block_size           brute-force loops + invariants (SGLang format)
silu_and_mul                   scipy ``expit`` closed form
gelu_and_mul                   ``torch.nn.functional.gelu`` (exact erf form,
                               library routine); Phi(1) known value; the
                               identity gelu(x) - gelu(-x) = x.  The routine is
                               sgl_kernel's ``gelu_and_mul`` (external).
swiglu                         reduces to ``torch.nn.functional.silu`` for
                               alpha = 1, no clamp, linear = 0; clamp and
                               interleaving checked against closed forms.  The
                               routine is triton_kernels' ``swiglu_fn``
                               (external, absent): *parity unpinned* (alpha /
                               limit / the +1 on the linear half follow the
                               published gpt-oss swiglu).
fused_experts (bf16)           fp64 per-token brute force; E=1/k=1 reduces to
                               a dense SwiGLU MLP (textbook routine); gelu
                               variant: E=1/k=1 dense GeGLU with torch's gelu
ep_localize                    identity map = no map; two ranks with disjoint
                               maps sum to the single-rank output (the EP
                               invariant); the map semantics is SGLang's
                               (external) expert_map: global -> local or -1
fused_experts_bias             fp64 per-token brute force; zero weights reduce
                               to sum_j w_j b2[e_j] (closed form).  The order
                               bias -> activation -> routing weight inside
                               matmul_ogs is *unpinned* (external code).
mxfp4_quant / mxfp4_dequant    torch's reference MX quantizer
                               (``torch.testing._internal.common_quantized.
                               to_mxfp``, RCEIL scale rule) bit for bit; the
                               OCP E2M1 table (16 codes) and tie / saturation
                               known answers; the MI355X hardware conversion
                               ``v_cvt_scalef32_pk_bf16_fp4`` (GPU test).  The
                               MXFP4 MoE GEMM itself = the bf16 path on
                               dequantized weights (pinned as above).
per_token_group_quant_fp8      torch ``float8_e4m3fn`` cast; exact powers of 2;
                               amax element maps to +-448 exactly
block_quant_fp8                same; dequant round-trip error bound
quant_int4 / dequant_int4      pack/unpack round trip; closed-form dequant of
                               constructed groups; error <= scale/2
fused_experts_fp8 / _w4a16     = fused_experts on dequantized operands, with the
                               quantization of activations restated; no
                               reference implementation exists (the reference
                               asserts ``use_fp8_w8a8 is False``,
                               ``ops/fused_moe.py:154``, and has no int4 path):
                               *parity to the reference unpinned*, pinned to
                               the dequantize-then-compute definition.
=============================  ===============================================
"""

from __future__ import annotations

import numpy as np
import torch

FP8_MAX = 448.0  # largest finite float8_e4m3fn value
FP8_EPS = 1e-10  # amax floor used before dividing by it
BLOCK_MS = (16, 32, 64, 128)  # tile heights triton_kernels.routing precomputes


# --------------------------------------------------------------------------
# routing: logits -> (topk_weights, topk_ids)
# --------------------------------------------------------------------------
def softmax_topk(logits: torch.Tensor, k: int, renormalize: bool = True):
    """softmax -> top-k -> renormalise.

    Follows ``tests/test_fused_moe.py:24-27`` (and the identical
    ``benchmark/test_fused_moe.py:15-17``).  Returns fp32 weights and int32
    ids, both ``[M, k]`` in descending-probability order.
    """
    p = torch.softmax(logits.float(), dim=-1)
    w, ids = torch.topk(p, k=k, dim=-1)
    if renormalize:
        w = w / w.sum(dim=-1, keepdim=True)
    return w, ids.to(torch.int32)


def grouped_topk(
    logits: torch.Tensor,
    k: int,
    n_group: int,
    topk_group: int,
    bias: torch.Tensor | None = None,
    renormalize: bool = True,
    scoring: str = "sigmoid",
):
    """DeepSeek-V3 style grouped top-k (SGLang ``biased_grouped_topk``).

    scores = sigmoid(logits) (or softmax); selection uses scores + bias;
    group score = sum of the top-2 biased scores of each group; keep the
    ``topk_group`` best groups; pick ``k`` experts among them by biased score;
    the returned weights are the *unbiased* scores of the chosen experts,
    renormalised.  The routed scaling factor is applied later, on the MoE
    output (``ops/fused_moe.py:399-404``).
    """
    M, E = logits.shape
    if scoring == "sigmoid":
        s = torch.sigmoid(logits.float())
    else:
        s = torch.softmax(logits.float(), dim=-1)
    sel = s if bias is None else s + bias.float()[None, :]
    g = sel.view(M, n_group, E // n_group)
    gs = g.topk(2, dim=-1).values.sum(dim=-1)  # [M, n_group]
    gidx = gs.topk(topk_group, dim=-1).indices
    gmask = torch.zeros_like(gs).scatter_(1, gidx, 1.0)
    emask = gmask[:, :, None].expand(M, n_group, E // n_group).reshape(M, E)
    masked = sel.masked_fill(emask == 0, float("-inf"))
    ids = masked.topk(k, dim=-1).indices
    w = s.gather(1, ids)
    if renormalize:
        w = w / w.sum(dim=-1, keepdim=True)
    return w, ids.to(torch.int32)


# --------------------------------------------------------------------------
# routing conversion / alignment (integer work: numpy)
# --------------------------------------------------------------------------
def standard_topk_to_routing(topk_weights, topk_ids, n_expts_tot: int):
    """Restates ``_standard_topk_to_triton_kernels`` (``ops/fused_moe.py:103-130``).

    * each token's k ids sorted ascending, weights gathered alongside (:114-117)
    * ``topk_indx`` = stable argsort of the flat sorted ids (:118): for every
      expert-sorted slot, the flat (token-major) index it came from
    * ``gate_indx`` = inverse permutation (:119)
    * ``gate_scal`` = weights in expert-sorted order (:120)
    * ``hist`` = per-expert counts (:121-123; histc over integer ids 0..E-1
      equals bincount)

    Returns a dict of numpy arrays (int32 / float32).
    """
    ids = np.asarray(topk_ids, dtype=np.int64)
    w = np.asarray(topk_weights, dtype=np.float32)
    M, k = ids.shape
    order = np.argsort(ids, axis=1, kind="stable")  # ids distinct per row
    expt_indx = np.take_along_axis(ids, order, axis=1).reshape(-1)
    expt_scal = np.take_along_axis(w, order, axis=1).reshape(-1)
    topk_indx = np.argsort(expt_indx, kind="stable")
    gate_indx = np.empty_like(topk_indx)
    gate_indx[topk_indx] = np.arange(M * k)
    hist = np.bincount(expt_indx, minlength=n_expts_tot)[:n_expts_tot]
    return dict(
        expt_indx=expt_indx.astype(np.int32),
        expt_scal=expt_scal.astype(np.float32),
        sort_order=order.astype(np.int32),
        topk_indx=topk_indx.astype(np.int32),
        gate_indx=gate_indx.astype(np.int32),
        gate_scal=expt_scal[topk_indx].astype(np.float32),
        hist=hist.astype(np.int32),
    )


def max_n_tiles(n_expts_tot: int, n_gates: int) -> int:
    """Tile-map length used by triton_kernels.routing (upstream, unpinned here).

    With n_gates <= E there is at most one tile per gate; otherwise every
    non-empty expert may waste one partial tile of the smallest block height.
    """
    if n_gates <= n_expts_tot:
        return n_gates
    m = min(BLOCK_MS)
    return n_expts_tot - 1 + -(-(n_gates - n_expts_tot + 1) // m)


def compute_expt_data(hist, n_expts_tot: int, n_gates: int, block_m: int):
    """ExptData for one tile height (``compute_expt_data_torch``, called at
    ``ops/fused_moe.py:124``; the routine lives in triton_kernels, absent).

    token_offs_raw = [0, cumsum(hist)]; token_offs_pad = [0, cumsum(ceil(hist /
    block_m))] (in tiles); block_pid_map[t] = (tile_in_expert << 16) | expert for
    used tiles, -1 for the rest.
    """
    hist = np.asarray(hist, dtype=np.int64)
    offs_raw = np.concatenate([[0], np.cumsum(hist)])
    ntl = (hist + block_m - 1) // block_m
    offs_pad = np.concatenate([[0], np.cumsum(ntl)])
    L = max_n_tiles(n_expts_tot, n_gates)
    pid = np.full(L, -1, dtype=np.int64)
    total = int(offs_pad[-1])
    if total:
        e_of = np.repeat(np.arange(n_expts_tot), ntl)
        blk = np.arange(total) - offs_pad[e_of]
        pid[:total] = (blk << 16) | e_of
    return dict(
        token_offs_raw=offs_raw.astype(np.int32),
        token_offs_pad=offs_pad.astype(np.int32),
        block_pid_map=pid.astype(np.int32),
        n_tiles=total,
    )


def moe_align_block_size(topk_ids, block_m: int, n_experts: int):
    """SGLang-format alignment (``moe_align_block_size``), the padded-tile
    view that the reference's ExptData encodes (``ops/fused_moe.py:124``).

    sorted_token_ids: flat indices into ``topk_ids`` (token * k + j, original
    column order), grouped by expert, ascending within an expert, each expert's
    run padded to a multiple of ``block_m`` with the sentinel ``M * k``.
    Length ``M*k + E*(block_m-1)``; entries past the padded total are sentinel.
    expert_ids: expert of each ``block_m`` block (-1 past the used blocks).
    num_tokens_post_padded: padded total.
    """
    ids = np.asarray(topk_ids, dtype=np.int64)
    M, k = ids.shape
    flat = ids.reshape(-1)
    n = M * k
    hist = np.bincount(flat, minlength=n_experts)[:n_experts]
    padded = (hist + block_m - 1) // block_m * block_m
    offs = np.concatenate([[0], np.cumsum(padded)])
    cap = n + n_experts * (block_m - 1)
    sorted_ids = np.full(cap, n, dtype=np.int64)
    order = np.argsort(flat, kind="stable")
    starts = np.concatenate([[0], np.cumsum(hist)])
    for e in range(n_experts):
        seg = order[starts[e]:starts[e + 1]]
        sorted_ids[offs[e]:offs[e] + len(seg)] = seg
    total = int(offs[-1])
    expert_ids = np.full(cap // block_m + 1, -1, dtype=np.int64)
    nb = total // block_m
    if nb:
        expert_ids[:nb] = np.repeat(np.arange(n_experts), padded // block_m)
    return dict(
        sorted_token_ids=sorted_ids.astype(np.int32),
        expert_ids=expert_ids.astype(np.int32),
        num_tokens_post_padded=np.int32(total),
    )


# --------------------------------------------------------------------------
# activation
# --------------------------------------------------------------------------
def silu_and_mul(inter: torch.Tensor) -> torch.Tensor:
    """``_silu_and_mul_kernel`` (``ops/fused_moe.py:28-47``): gate = first half,
    up = second half, ``gate / (1 + exp(-gate)) * up`` in fp32, stored in the
    dtype of the output buffer (bf16 in the reference, :198-202)."""
    h = inter.shape[-1] // 2
    g = inter[..., :h].float()
    u = inter[..., h:].float()
    return (g / (1.0 + torch.exp(-g))) * u


def gelu_and_mul(inter: torch.Tensor) -> torch.Tensor:
    """``gelu_and_mul`` (sgl_kernel, called at ``ops/fused_moe.py:19-21,203-204``):
    gate = first half, up = second half, exact (erf) GELU of the gate times
    up, in fp32."""
    h = inter.shape[-1] // 2
    g = inter[..., :h].double()
    u = inter[..., h:].double()
    erf = torch.special.erf(g / np.sqrt(2.0))
    return (0.5 * g * (1.0 + erf) * u).float()


def swiglu(inter: torch.Tensor, alpha: float = 1.0, limit: float | None = None) -> torch.Tensor:
    """The fused activation of the bias path (``ops/fused_moe.py:258-259``,
    triton_kernels ``swiglu_fn``): columns interleaved, gate = even, linear =
    odd; ``g = min(gate, limit)``, ``l = clamp(linear, -limit, limit)`` when a
    limit is given; ``g * sigmoid(alpha * g) * (l + 1)`` in fp32."""
    g = inter[..., 0::2].double()
    lin = inter[..., 1::2].double()
    if limit is not None and limit > 0:
        g = torch.clamp(g, max=limit)
        lin = torch.clamp(lin, min=-limit, max=limit)
    return (g / (1.0 + torch.exp(-alpha * g)) * (lin + 1.0)).float()


# --------------------------------------------------------------------------
# fused experts (bf16 semantics)
# --------------------------------------------------------------------------
def _expert_groups(r, k):
    """Yield (expert, slot range, token ids) in expert order."""
    hist = r["hist"]
    offs = np.concatenate([[0], np.cumsum(hist)])
    for e in range(len(hist)):
        a, b = int(offs[e]), int(offs[e + 1])
        if a == b:
            continue
        yield e, a, b, r["topk_indx"][a:b] // k


def fused_experts(
    x: torch.Tensor,
    w13: torch.Tensor,
    w2: torch.Tensor,
    topk_weights,
    topk_ids,
    apply_router_weight_on_input: bool = False,
    routed_scaling_factor: float | None = None,
    w13_deq=None,
    w2_deq=None,
    act_quant=None,
    a1_deq=None,
    activation: str = "silu",
):
    """Fused MoE forward, ``triton_kernel_fused_experts`` (``ops/fused_moe.py:181-216``).

    Weights are in SGLang layer layout: ``w13 [E, 2N, K]``, ``w2 [E, K, N]``
    (the reference transposes them per call at :326-327 into matmul_ogs's
    ``[E, K, 2N]`` / ``[E, N, K]``; the product is the same).

    Rounding points follow the reference: GEMM1 accumulates in fp32 and its
    output ``intermediate`` is bf16 (matmul_ogs output dtype = input dtype);
    silu·mul reads bf16 and writes bf16 (:198-202); GEMM2 rows are scaled by
    ``gate_scal`` (:187) and summed over the k slots of a token in fp32, the
    result stored as bf16 (:216).  ``routed_scaling_factor`` multiplies the
    combined output (:399-404).

    ``w13_deq``/``w2_deq`` (callables e -> fp32 matrix) and ``act_quant`` /
    ``a1_deq`` let the fp8 / int4 oracles reuse this with dequantized operands.
    ``activation``: "silu" (``_silu_and_mul_triton``) or "gelu"
    (``gelu_and_mul``), the branch at :198-206.
    """
    act_fn = {"silu": silu_and_mul, "gelu": gelu_and_mul}[activation]
    M, K = x.shape
    k = topk_ids.shape[1]
    E = w13.shape[0] if w13 is not None else w13_deq.E
    r = standard_topk_to_routing(topk_weights, topk_ids, E)
    xin = a1_deq if a1_deq is not None else x.float()
    y = torch.zeros(M * k, K, dtype=torch.float32)
    gate_scal = torch.from_numpy(r["gate_scal"])
    for e, a, b, tok in _expert_groups(r, k):
        tok = torch.from_numpy(tok.astype(np.int64))
        W1 = w13_deq(e) if w13_deq is not None else w13[e].float()
        W2 = w2_deq(e) if w2_deq is not None else w2[e].float()
        inter = xin[tok] @ W1.t()
        if apply_router_weight_on_input:
            inter = inter * gate_scal[a:b, None]
        inter = inter.to(torch.bfloat16)
        act = act_fn(inter).to(torch.bfloat16).float()
        if act_quant is not None:
            act = act_quant(act)
        out = act @ W2.t()
        if not apply_router_weight_on_input:
            out = out * gate_scal[a:b, None]
        flat = torch.from_numpy(r["topk_indx"][a:b].astype(np.int64))
        y[flat] = out
    res = y.view(M, k, K).sum(dim=1)
    if routed_scaling_factor is not None and routed_scaling_factor != 1.0:
        res = res * routed_scaling_factor
    return res.to(torch.bfloat16)


def ep_localize(topk_weights, topk_ids, expert_map):
    """Expert parallel (the ``expert_map`` / ``global_num_experts`` arguments,
    ``ops/fused_moe.py:145-146,160``): ``expert_map [n_global]`` maps a global
    expert id to a local one or -1.  Returns routing for the local experts in
    which every non-local choice points at local expert 0 with weight 0, so it
    contributes exactly 0 (silu(0)·0 = 0 also when the weight multiplies the
    input)."""
    emap = torch.as_tensor(expert_map).long()
    ids = torch.as_tensor(topk_ids).long()
    ok = (ids >= 0) & (ids < emap.numel())
    loc = torch.where(ok, emap[ids.clamp(0, emap.numel() - 1)], torch.full_like(ids, -1))
    keep = loc >= 0
    tw = torch.where(keep, torch.as_tensor(topk_weights).float(), torch.zeros(()))
    return tw, torch.where(keep, loc, torch.zeros_like(loc)).to(torch.int32)


def fused_experts_bias(x, w13, b13, w2, b2, topk_weights, topk_ids,
                       apply_router_weight_on_input: bool = False, alpha: float = 1.0,
                       limit: float | None = None):
    """``triton_kernel_fused_experts_with_bias`` (``ops/fused_moe.py:219-309``),
    SGLang layouts ``w13 [E, 2N, K]`` with interleaved gate / linear rows,
    ``b13 [E, 2N]``, ``w2 [E, K, N]``, ``b2 [E, K]``.  GEMM1 (fp32 accumulate)
    + bias -> swiglu in fp32 (fused into matmul_ogs, no bf16 rounding of the
    GEMM1 result) -> routing weight when applied on the input -> bf16; GEMM2
    (fp32) + bias -> routing weight otherwise; top-k sum in fp32 -> bf16."""
    M, K = x.shape
    k = topk_ids.shape[1]
    E = w13.shape[0]
    r = standard_topk_to_routing(topk_weights, topk_ids, E)
    xin = x.float()
    y = torch.zeros(M * k, K, dtype=torch.float32)
    gate_scal = torch.from_numpy(r["gate_scal"])
    for e, a, b, tok in _expert_groups(r, k):
        tok = torch.from_numpy(tok.astype(np.int64))
        inter = xin[tok] @ w13[e].float().t() + b13[e].float()
        act = swiglu(inter, alpha, limit)
        if apply_router_weight_on_input:
            act = act * gate_scal[a:b, None]
        act = act.to(torch.bfloat16).float()
        out = act @ w2[e].float().t() + b2[e].float()
        if not apply_router_weight_on_input:
            out = out * gate_scal[a:b, None]
        flat = torch.from_numpy(r["topk_indx"][a:b].astype(np.int64))
        y[flat] = out
    return y.view(M, k, K).sum(dim=1).to(torch.bfloat16)


def fused_experts_bias_bruteforce(x, w13, b13, w2, b2, topk_weights, topk_ids, alpha=1.0,
                                  limit=None):
    """Second oracle for the bias path: per-token, per-slot loop in fp64."""
    M, K = x.shape
    N = w2.shape[2]
    xd = x.double()
    out = torch.zeros(M, K, dtype=torch.float64)
    for t in range(M):
        for j in range(topk_ids.shape[1]):
            e = int(topk_ids[t, j])
            h = w13[e].double() @ xd[t] + b13[e].double()
            g, lin = h[0::2], h[1::2]
            if limit is not None and limit > 0:
                g = g.clamp(max=limit)
                lin = lin.clamp(-limit, limit)
            a = g * torch.sigmoid(alpha * g) * (lin + 1.0)
            out[t] += float(topk_weights[t, j]) * (w2[e].double() @ a + b2[e].double())
    assert out.shape[1] == K and N * 2 == w13.shape[1]
    return out


def fused_experts_bruteforce(x, w13, w2, topk_weights, topk_ids):
    """Second oracle: per-token, per-slot loop in fp64, no routing conversion.

    out[t] = sum_j w[t,j] * (silu(x W1g_e) * (x W1u_e)) @ W2_e^T with e =
    ids[t,j].  Rounding points are not modelled (fp64 throughout).
    """
    M, K = x.shape
    N = w2.shape[2]
    xd = x.double()
    out = torch.zeros(M, K, dtype=torch.float64)
    for t in range(M):
        for j in range(topk_ids.shape[1]):
            e = int(topk_ids[t, j])
            w1 = w13[e].double()
            g = w1[:N] @ xd[t]
            u = w1[N:] @ xd[t]
            a = g * torch.sigmoid(g) * u
            out[t] += float(topk_weights[t, j]) * (w2[e].double() @ a)
    return out


# --------------------------------------------------------------------------
# fp8 e4m3 (OCP) block quantization — SGLang fused_experts(use_fp8_w8a8=True,
# block_shape=[128, 128]) contract; no reference implementation.
# --------------------------------------------------------------------------
def per_token_group_quant_fp8(x: torch.Tensor, group: int = 128):
    """Dynamic 1 x group activation quant: scale = max(amax, eps) / 448,
    q = clamp(x / scale, +-448) cast to float8_e4m3fn (round to nearest even).
    Returns (q [M, K] float8_e4m3fn, scale [M, K/group] fp32)."""
    M, K = x.shape
    xf = x.float().view(M, K // group, group)
    amax = xf.abs().amax(dim=-1).clamp_min(FP8_EPS)
    s = amax / FP8_MAX
    q = (xf / s[..., None]).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return q.view(M, K), s


def dequant_token_group(q, s, group: int = 128):
    M, K = q.shape
    return (q.float().view(M, K // group, group) * s[..., None]).view(M, K)


def block_quant_fp8(w: torch.Tensor, block=(128, 128)):
    """Per-block weight quant of ``w [E, R, C]``: scale[e, i, j] = amax / 448
    over rows i*bR.. and cols j*bC..; returns (q float8_e4m3fn, scale fp32
    [E, R/bR, C/bC])."""
    E, R, C = w.shape
    bR, bC = block
    wf = w.float().view(E, R // bR, bR, C // bC, bC)
    amax = wf.abs().amax(dim=(2, 4)).clamp_min(FP8_EPS)
    s = amax / FP8_MAX
    q = (wf / s[:, :, None, :, None]).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return q.view(E, R, C), s


def dequant_block(q_e, s_e, block=(128, 128)):
    """Dequantize one expert's ``[R, C]`` block-quantized matrix to fp32."""
    R, C = q_e.shape
    bR, bC = block
    return (q_e.float().view(R // bR, bR, C // bC, bC) * s_e[:, None, :, None]).view(R, C)


class _Deq:
    def __init__(self, fn, E):
        self.fn, self.E = fn, E

    def __call__(self, e):
        return self.fn(e)


def fused_experts_fp8(x, w13_q, w13_s, w2_q, w2_s, topk_weights, topk_ids,
                      routed_scaling_factor=None, block=(128, 128)):
    """W8A8 block-scale fused MoE: x is quantized per 1x128 token group, GEMM1
    runs on dequantized operands, the bf16 activation is re-quantized per 1x128
    group before GEMM2 (SGLang's fp8 block path)."""
    g = block[1]
    q, s = per_token_group_quant_fp8(x, g)
    a1 = dequant_token_group(q, s, g)

    def aq(act):
        qq, ss = per_token_group_quant_fp8(act, g)
        return dequant_token_group(qq, ss, g)

    E = w13_q.shape[0]
    return fused_experts(
        x, None, None, topk_weights, topk_ids,
        routed_scaling_factor=routed_scaling_factor,
        w13_deq=_Deq(lambda e: dequant_block(w13_q[e], w13_s[e], block), E),
        w2_deq=_Deq(lambda e: dequant_block(w2_q[e], w2_s[e], block), E),
        act_quant=aq, a1_deq=a1,
    )


# --------------------------------------------------------------------------
# int4 W4A16 (asymmetric uint4, group along the reduction dim)
# --------------------------------------------------------------------------
def quant_int4(w: torch.Tensor, group: int = 128):
    """Asymmetric uint4 quant of ``w [E, R, C]`` in groups of ``group`` along C
    (C is the reduction dim, R the output rows).

    scale = (max - min) / 15 rounded to fp16 (floored at 1e-8 before rounding),
    zero = clamp(round(-min / scale), 0, 15), q = clamp(round(w / scale) + zero,
    0, 15); dequant w' = (q - zero) * scale.

    Layout (group-major scales/zeros as in AWQ checkpoints, weights packed along
    the reduction dim):
      qweight ``[E, R, C/2] uint8``: element 2i in the low nibble, 2i+1 high;
      scales  ``[E, G, R] fp16`` with G = C / group;
      zeros   ``[E, G, ceil(R/2)] uint8``: row 2j low nibble, row 2j+1 high.
    """
    E, R, C = w.shape
    G = C // group
    wf = w.float().view(E, R, G, group)
    mn = wf.amin(dim=-1)
    mx = wf.amax(dim=-1)
    sc = ((mx - mn) / 15.0).clamp_min(1e-8).to(torch.float16)
    scf = sc.float()
    z = torch.clamp(torch.round(-mn / scf), 0, 15)
    q = torch.clamp(torch.round(wf / scf[..., None]) + z[..., None], 0, 15).to(torch.uint8)
    q = q.view(E, R, C)
    zeros = pack_u4(z.to(torch.uint8).transpose(1, 2).contiguous())
    return pack_u4(q), sc.transpose(1, 2).contiguous(), zeros


def pack_u4(q: torch.Tensor) -> torch.Tensor:
    """Pack uint4 values (uint8 tensor, last dim) two per byte, low nibble first."""
    n = q.shape[-1]
    if n % 2:
        q = torch.cat([q, torch.zeros(*q.shape[:-1], 1, dtype=torch.uint8)], dim=-1)
    lo = q[..., 0::2]
    hi = q[..., 1::2]
    return (lo | (hi << 4)).contiguous()


def unpack_u4(p: torch.Tensor, n: int) -> torch.Tensor:
    lo = p & 0xF
    hi = p >> 4
    out = torch.stack([lo, hi], dim=-1).view(*p.shape[:-1], p.shape[-1] * 2)
    return out[..., :n]


def dequant_int4(qw_e, sc_e, z_e, group: int = 128):
    """One expert: packed ``[R, C/2]``, scales ``[G, R]``, zeros ``[G, ceil(R/2)]``
    -> fp32 ``[R, C]`` via (q - zero) * scale."""
    R = qw_e.shape[0]
    C = qw_e.shape[1] * 2
    G = C // group
    q = unpack_u4(qw_e, C).float().view(R, G, group)
    z = unpack_u4(z_e, R).float().t()  # [R, G]
    return ((q - z[..., None]) * sc_e.float().t()[..., None]).view(R, C)


def fused_experts_w4a16(x, w13_q, w13_sc, w13_z, w2_q, w2_sc, w2_z,
                        topk_weights, topk_ids, group=128, routed_scaling_factor=None):
    """W4A16: bf16 activations, int4 weights dequantized to fp32; otherwise the
    bf16 fused_experts semantics (same rounding points)."""
    E = w13_q.shape[0]
    return fused_experts(
        x, None, None, topk_weights, topk_ids,
        routed_scaling_factor=routed_scaling_factor,
        w13_deq=_Deq(lambda e: dequant_int4(w13_q[e], w13_sc[e], w13_z[e], group), E),
        w2_deq=_Deq(lambda e: dequant_int4(w2_q[e], w2_sc[e], w2_z[e], group), E),
    )


# --------------------------------------------------------------------------
# seeded input generator (reference rule: seed = M+K+N+E+topk,
# tests/test_fused_moe.py:50-58; layouts / scales from the BASELINE configs)
# --------------------------------------------------------------------------
def make_inputs(M, K, N, E, topk, wscale=0.02, seed=None, routing="softmax",
                expert_bias_std=0.0, n_group=8, topk_group=4, dtype=torch.bfloat16):
    """x ~ N(0,1), w13 [E,2N,K] and w2 [E,K,N] ~ N(0, wscale), router logits
    ~ N(0,1) (+ per-expert bias ~ N(0, expert_bias_std)).  Generated on CPU so
    the GPU and the oracle see identical bits."""
    s = M + K + N + E + topk if seed is None else seed
    g = torch.Generator().manual_seed(s)
    x = torch.randn(M, K, generator=g).to(dtype)
    w13 = (torch.randn(E, 2 * N, K, generator=g) * wscale).to(dtype)
    w2 = (torch.randn(E, K, N, generator=g) * wscale).to(dtype)
    logits = torch.randn(M, E, generator=g)
    if expert_bias_std:
        g2 = torch.Generator().manual_seed(s + 1)
        logits = logits + torch.randn(E, generator=g2)[None, :] * expert_bias_std
    if routing == "softmax":
        tw, ti = softmax_topk(logits, topk)
    else:
        tw, ti = grouped_topk(logits, topk, n_group, topk_group)
    return dict(x=x, w13=w13, w2=w2, logits=logits, topk_weights=tw, topk_ids=ti)


# --------------------------------------------------------------------------
# MXFP4 weights (OCP Microscaling Formats v1.0: E2M1 elements, one E8M0
# scale per 32 consecutive elements along the reduction dim).  The reference
# passes such weights to matmul_ogs through ``w1_pcg`` / ``w2_pcg``
# (ops/fused_moe.py:219-309, :374-378) with bf16 activations (W4A16).
# --------------------------------------------------------------------------
E2M1_VALUES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float32)


def e2m1_encode(v: np.ndarray) -> np.ndarray:
    """fp32 -> E2M1 code (bit 3 = sign): round to nearest, ties to the even
    code, saturating at 6."""
    a = np.abs(v.astype(np.float32))
    c = np.zeros(a.shape, dtype=np.uint8)
    c = np.where(a > 0.25, 1, c)
    c = np.where(a >= 0.75, 2, c)
    c = np.where(a > 1.25, 3, c)
    c = np.where(a >= 1.75, 4, c)
    c = np.where(a > 2.5, 5, c)
    c = np.where(a >= 3.5, 6, c)
    c = np.where(a > 5.0, 7, c)
    return (c | (np.signbit(v).astype(np.uint8) << 3)).astype(np.uint8)


def e2m1_decode(c: np.ndarray) -> np.ndarray:
    v = E2M1_VALUES[c & 7]
    return np.where(c & 8, -v, v).astype(np.float32)


def e8m0_value(s: np.ndarray) -> np.ndarray:
    """E8M0 scale byte -> 2^(s - 127) (255 = NaN)."""
    s = s.astype(np.int32)
    v = np.ldexp(np.float32(1.0), np.minimum(s, 254) - 127)  # 255 (NaN) handled below
    return np.where(s == 255, np.float32(np.nan), v).astype(np.float32)


def mxfp4_quant(w: torch.Tensor, block: int = 32):
    """``w [..., C]`` (bf16) -> (packed e2m1 ``[..., C/2]`` u8, element 2i in the
    low nibble; e8m0 scales ``[..., C/32]`` u8), with the scale rule of torch's
    reference MX quantizer (RCEIL): exponent = ceil(log2(amax / 6)) clamped to
    [-127, 127], so no element saturates, and elements x * 2^-exponent rounded
    to E2M1 (nearest, ties to even)."""
    wf = w.float().numpy()
    *lead, C = wf.shape
    g = wf.reshape(*lead, C // block, block)
    amax = np.abs(g).max(axis=-1)
    with np.errstate(divide="ignore"):
        ex = np.ceil(np.log2(amax / np.float32(6.0)))
    ex = np.clip(np.where(np.isfinite(ex), ex, -127), -127, 127).astype(np.int32)
    s = (ex + 127).astype(np.uint8)
    inv = np.where(s == 0, np.float32(1.0), np.ldexp(np.float32(1.0), -ex)).astype(np.float32)
    codes = e2m1_encode(g * inv[..., None]).reshape(*lead, C)
    packed = (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)
    return torch.from_numpy(packed), torch.from_numpy(s)


def mxfp4_dequant(packed: torch.Tensor, scales: torch.Tensor, block: int = 32) -> torch.Tensor:
    """Inverse layout of ``mxfp4_quant``: value = e2m1 * 2^(scale - 127), fp32."""
    p = packed.numpy()
    codes = np.empty((*p.shape[:-1], p.shape[-1] * 2), dtype=np.uint8)
    codes[..., 0::2] = p & 15
    codes[..., 1::2] = p >> 4
    v = e2m1_decode(codes)
    sv = np.repeat(e8m0_value(scales.numpy()), block, axis=-1)
    return torch.from_numpy(v * sv)


def fused_experts_mxfp4(x, w13_q, w13_s, w2_q, w2_s, topk_weights, topk_ids,
                        routed_scaling_factor=None, apply_router_weight_on_input=False,
                        activation="silu"):
    """MXFP4 weights (SGLang layout, ``[E, rows, K/2]`` + ``[E, rows, K/32]``),
    bf16 activations: the bf16 fused_experts semantics on dequantized weights."""
    E = w13_q.shape[0]
    return fused_experts(
        x, None, None, topk_weights, topk_ids,
        apply_router_weight_on_input=apply_router_weight_on_input,
        routed_scaling_factor=routed_scaling_factor, activation=activation,
        w13_deq=_Deq(lambda e: mxfp4_dequant(w13_q[e], w13_s[e]), E),
        w2_deq=_Deq(lambda e: mxfp4_dequant(w2_q[e], w2_s[e]), E),
    )
