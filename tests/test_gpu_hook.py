"""The SGLang hook ``fused_moe_flagos`` (ref ops/fused_moe.py:312-406) and the
``no_combine`` outputs, on the GPU through the C ABI, against the oracle.

* plain bf16 and fp8 block-scale layers, ``routed_scaling_factor`` applied
  after the combine (:399-404) and not under ``no_combine``;
* triton_kernels-format routing recognised by its fields, whatever class
  carries them (SGLang's ``TritonKernelTopKOutput`` named tuple of foreign
  ``RoutingData`` / ``GatherIndx`` / ``ScatterIndx`` objects);
* ``no_combine`` row order: ``fused_experts`` (SGLang ``fused_experts``
  contract) returns slot ``(t, j)`` = the choice ``topk_ids[t, j]``;
  ``triton_kernel_fused_experts(scatter_indx=None)`` returns the routing's
  flat order (each token's experts ascending); slots whose expert an
  expert map drops are zero.
"""

from collections import namedtuple
from types import SimpleNamespace

import pytest
import torch

import flaggems_sglang
from flaggems_sglang import quant as Q
from flaggems_sglang.ops import fused_moe as F
from oracle import fused_moe_oracle as O

from test_gpu_fused_moe import _close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _per_slot_oracle(d, ids, weights, w13=None, w2=None, **kw):
    """[M, k, K]: slot (t, j) alone, i.e. the k=1 oracle on column j."""
    w13 = d["w13"] if w13 is None else w13
    w2 = d["w2"] if w2 is None else w2
    cols = [O.fused_experts(d["x"], w13, w2, weights[:, j:j + 1], ids[:, j:j + 1], **kw)
            for j in range(ids.shape[1])]
    return torch.stack(cols, dim=1)


def _hook_objects(d, E, no_combine=False, rsf=None, on_input=False, topk_output=None):
    cfg = SimpleNamespace(num_experts=E, no_combine=no_combine, activation="silu",
                          apply_router_weight_on_input=on_input, routed_scaling_factor=rsf)
    obj = SimpleNamespace(runner=SimpleNamespace(config=cfg))
    if topk_output is None:
        topk_output = SimpleNamespace(topk_weights=d["topk_weights"].to(DEV),
                                      topk_ids=d["topk_ids"].to(DEV))
    disp = SimpleNamespace(hidden_states=d["x"].to(DEV), topk_output=topk_output)
    return obj, disp


def _bf16_layer(d):
    layer = torch.nn.Module()
    layer.register_parameter("w13_weight", torch.nn.Parameter(d["w13"].to(DEV), requires_grad=False))
    layer.register_parameter("w2_weight", torch.nn.Parameter(d["w2"].to(DEV), requires_grad=False))
    return layer


def _fp8_layer(d):
    q1, s1 = Q.quantize_fp8_block(d["w13"].to(DEV))
    q2, s2 = Q.quantize_fp8_block(d["w2"].to(DEV))
    layer = torch.nn.Module()
    for n, t in (("w13_weight", q1), ("w2_weight", q2), ("w13_weight_scale_inv", s1),
                 ("w2_weight_scale_inv", s2)):
        layer.register_parameter(n, torch.nn.Parameter(t, requires_grad=False))
    return layer, (q1, s1, q2, s2)


@pytest.mark.parametrize("M", [3, 200])
@pytest.mark.parametrize("rsf", [None, 2.5])
def test_hook_bf16_layer(M, rsf):
    E, k = 8, 2
    d = O.make_inputs(M, 256, 384, E, k, wscale=0.05)
    obj, disp = _hook_objects(d, E, rsf=rsf)
    out = F.fused_moe_flagos(obj, _bf16_layer(d), disp).hidden_states
    ref = O.fused_experts(d["x"], d["w13"], d["w2"], d["topk_weights"], d["topk_ids"],
                          routed_scaling_factor=rsf)
    _close(out, ref, 2e-2)


@pytest.mark.parametrize("M", [3, 200])
def test_hook_fp8_layer_routed_scaling(M):
    E, k = 8, 4
    d = O.make_inputs(M, 512, 256, E, k, wscale=0.02)
    layer, (q1, s1, q2, s2) = _fp8_layer(d)
    obj, disp = _hook_objects(d, E, rsf=2.5)
    out = F.fused_moe_flagos(obj, layer, disp).hidden_states
    ref = O.fused_experts_fp8(d["x"], q1.cpu(), s1.cpu(), q2.cpu(), s2.cpu(), d["topk_weights"],
                              d["topk_ids"], routed_scaling_factor=2.5)
    _close(out, ref, 5e-2)


@pytest.mark.parametrize("fp8", [False, True])
def test_hook_no_combine(fp8):
    """no_combine through the hook: [M, k, K] in topk_ids column order, no
    routed scaling."""
    M, E, k = 37, 8, 2
    d = O.make_inputs(M, 512, 256, E, k, wscale=0.02)
    if fp8:
        layer, (q1, s1, q2, s2) = _fp8_layer(d)
    else:
        layer = _bf16_layer(d)
    obj, disp = _hook_objects(d, E, no_combine=True, rsf=2.5)
    out = F.fused_moe_flagos(obj, layer, disp).hidden_states
    assert out.shape == (M, k, 512)
    if fp8:
        cols = [O.fused_experts_fp8(d["x"], q1.cpu(), s1.cpu(), q2.cpu(), s2.cpu(),
                                    d["topk_weights"][:, j:j + 1], d["topk_ids"][:, j:j + 1])
                for j in range(k)]
        _close(out, torch.stack(cols, 1), 5e-2)
    else:
        _close(out, _per_slot_oracle(d, d["topk_ids"], d["topk_weights"]), 2e-2)


# Foreign containers with the triton_kernels field names (not this package's classes)
TritonKernelTopKOutput = namedtuple("TritonKernelTopKOutput", "routing_data gather_indx scatter_indx")


class _ForeignRoutingData:
    def __init__(self, gate_scal, expt_hist, n_expts_tot, n_expts_act, expt_data):
        self.gate_scal, self.expt_hist = gate_scal, expt_hist
        self.n_expts_tot, self.n_expts_act, self.expt_data = n_expts_tot, n_expts_act, expt_data


def _foreign_triple(tw, ti, E):
    rd, gi, si = F._standard_topk_to_triton_kernels(tw, ti, E)
    # upstream ExptData: offsets and per-block_m dicts, no n_tiles
    ed = SimpleNamespace(hist=rd.expt_hist, token_offs_raw=rd.expt_data.token_offs_raw,
                         token_offs_pad={}, block_pid_map={})
    frd = _ForeignRoutingData(rd.gate_scal, rd.expt_hist, rd.n_expts_tot, rd.n_expts_act, ed)
    return TritonKernelTopKOutput(frd, SimpleNamespace(src_indx=gi.src_indx, dst_indx=gi.dst_indx),
                                  SimpleNamespace(src_indx=si.src_indx, dst_indx=si.dst_indx))


@pytest.mark.parametrize("M", [5, 300])
def test_hook_foreign_triton_routing(M):
    E, k = 16, 4
    d = O.make_inputs(M, 256, 384, E, k, wscale=0.05)
    trip = _foreign_triple(d["topk_weights"].to(DEV), d["topk_ids"].to(DEV), E)
    assert not isinstance(trip.routing_data, F.RoutingData)
    obj, disp = _hook_objects(d, E, rsf=1.5, topk_output=trip)
    out = F.fused_moe_flagos(obj, _bf16_layer(d), disp).hidden_states
    ref = O.fused_experts(d["x"], d["w13"], d["w2"], d["topk_weights"], d["topk_ids"],
                          routed_scaling_factor=1.5)
    _close(out, ref, 2e-2)
    # the foreign ExptData is left as it came
    assert trip.routing_data.expt_data.block_pid_map == {}


def test_reference_api_no_combine_flat_order():
    """triton_kernel_fused_experts(scatter_indx=None): [M, k, K], slot (t, r)
    = token t's r-th expert in ascending id order (the routing's expt_indx)."""
    M, K, N, E, k = 29, 256, 384, 8, 3
    d = O.make_inputs(M, K, N, E, k, wscale=0.05)
    tw, ti = d["topk_weights"].to(DEV), d["topk_ids"].to(DEV)
    rd, gi, _ = F._standard_topk_to_triton_kernels(tw, ti, E)
    out = flaggems_sglang.triton_kernel_fused_experts(
        d["x"].to(DEV), d["w13"].transpose(1, 2).to(DEV), d["w2"].transpose(1, 2).to(DEV), rd, gi, None)
    assert out.shape == (M, k, K)
    ids_s, order = torch.sort(d["topk_ids"].long(), dim=1)
    w_s = torch.gather(d["topk_weights"], 1, order)
    _close(out, _per_slot_oracle(d, ids_s.to(torch.int32), w_s), 2e-2)


@pytest.mark.parametrize("M", [40, 300])
def test_no_combine_with_dropped_experts(M):
    """no_combine + expert_map: the slots of non-local experts are zero, the
    others match the per-slot oracle (previously an out-of-range gather)."""
    K, N, E, k = 256, 384, 8, 2
    d = O.make_inputs(M, K, N, E, k, wscale=0.05)
    emap = torch.arange(E, dtype=torch.int32)
    emap[3] = -1
    emap[4:] -= 1                      # local experts 0..6 = global 0,1,2,4,..,7
    keep = [e for e in range(E) if e != 3]
    lw13, lw2 = d["w13"][keep].contiguous(), d["w2"][keep].contiguous()
    out = flaggems_sglang.fused_experts(d["x"].to(DEV), lw13.to(DEV), lw2.to(DEV),
                                        d["topk_weights"].to(DEV), d["topk_ids"].to(DEV),
                                        no_combine=True, expert_map=emap.to(DEV),
                                        global_num_experts=E)
    assert out.shape == (M, k, K)
    dropped = d["topk_ids"] == 3
    assert dropped.any()
    assert torch.count_nonzero(out[dropped.to(DEV)]) == 0
    ltw, lti = O.ep_localize(d["topk_weights"], d["topk_ids"], emap)
    _close(out, _per_slot_oracle(d, lti, ltw, w13=lw13, w2=lw2), 2e-2)
