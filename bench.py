#!/usr/bin/env python
"""Fused-MoE benchmark on one MI355X.

Headline (``value``): Mixtral-8x7B-shape bf16 fused MoE at M=4096 tokens
(prefill), whole op per step = alignment + GEMM1+SiLU +
GEMM2 + top-k sum, inputs (x, weights, top-k routing) resident in HBM.
Unit TFLOP/s with FLOPs = 6*M*k*K*N.

Also on the same line:
  roofline      dominant kernel (GEMM1+SiLU) timed with HIP events on the
                launch stream over its own measured loop;
  cpu_baseline  the CPU oracle (a restatement of the reference, fp32 torch on
                the host cores) on a bounded token sample of the same workload;
  secondary     north-star points: DeepSeek-V3-shape fp8 W8A8 at M=4096
                (prefill, % fp8 MFMA peak and % of min(peak, AI*BW)) and
                Mixtral-shape W4A16 decode at M in {1, 4, 16, 64} (tiled int4
                weights; M=1 / 16 also row-major), % HBM peak; plus DSV3 at
                M=1 / 128 and Qwen3 at M=64 / 8192 (the other BASELINE configs).

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
"""

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "flaggems-sglang_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK = {"bf16": 2500.0, "fp8": 5000.0, "hbm_gbs": 8000.0}  # MI355X dense TFLOP/s, GB/s

WORKLOADS = {
    # name: (M, K, N, E, k, wtype, routing)
    "mixtral_bf16_m4096": (4096, 4096, 14336, 8, 2, "bf16", "softmax"),
    "mixtral_bf16_m1": (1, 4096, 14336, 8, 2, "bf16", "softmax"),
    "mixtral_bf16_m16": (16, 4096, 14336, 8, 2, "bf16", "softmax"),
    "mixtral_bf16_m256": (256, 4096, 14336, 8, 2, "bf16", "softmax"),
    "tiny_bf16_m64": (64, 128, 256, 8, 2, "bf16", "softmax"),
    "qwen3_bf16_m1": (1, 2048, 768, 128, 8, "bf16", "softmax_bias"),
    "qwen3_bf16_m1024": (1024, 2048, 768, 128, 8, "bf16", "softmax_bias"),
    "qwen3_bf16_m8192": (8192, 2048, 768, 128, 8, "bf16", "softmax_bias"),
    "dsv3_fp8_m4096": (4096, 7168, 2048, 256, 8, "fp8", "grouped"),
    "dsv3_fp8_m8192": (8192, 7168, 2048, 256, 8, "fp8", "grouped"),
    "dsv3_fp8_m1": (1, 7168, 2048, 256, 8, "fp8", "grouped"),
    "dsv3_fp8_m128": (128, 7168, 2048, 256, 8, "fp8", "grouped"),
    "qwen3_bf16_m64": (64, 2048, 768, 128, 8, "bf16", "softmax_bias"),
    "mixtral_w4a16_m1": (1, 4096, 14336, 8, 2, "int4", "softmax"),
    "mixtral_w4a16_m16": (16, 4096, 14336, 8, 2, "int4", "softmax"),
    # the same int4 weights tiled at load time (quant.tile_int4)
    "mixtral_w4a16t_m1": (1, 4096, 14336, 8, 2, "int4t", "softmax"),
    "mixtral_w4a16t_m16": (16, 4096, 14336, 8, 2, "int4t", "softmax"),
    "mixtral_w4a16t_m4": (4, 4096, 14336, 8, 2, "int4t", "softmax"),
    "mixtral_w4a16t_m64": (64, 4096, 14336, 8, 2, "int4t", "softmax"),
    "mixtral_w4a16t_m256": (256, 4096, 14336, 8, 2, "int4t", "softmax"),
    "mixtral_w4a16t_m4096": (4096, 4096, 14336, 8, 2, "int4t", "softmax"),
    # OCP MXFP4 weights (e2m1 + e8m0 per 32), bf16 activations
    "mixtral_mxfp4_m1": (1, 4096, 14336, 8, 2, "mxfp4", "softmax"),
    "mixtral_mxfp4_m16": (16, 4096, 14336, 8, 2, "mxfp4", "softmax"),
    "mixtral_mxfp4t_m1": (1, 4096, 14336, 8, 2, "mxfp4t", "softmax"),
    "mixtral_mxfp4t_m16": (16, 4096, 14336, 8, 2, "mxfp4t", "softmax"),
}
# the reference's own benchmark sweep (benchmark/attri_util.py:45-56):
# K=1280, N=3072, E=64, top-8, bf16
for _m in (1, 4, 17, 64, 1024, 2048, 4096):
    WORKLOADS[f"refsweep_bf16_m{_m}"] = (_m, 1280, 3072, 64, 8, "bf16", "softmax")

# every BASELINE.json point besides the headline, then the reference's sweep
DEFAULT_SECONDARY = (
    "dsv3_fp8_m4096,dsv3_fp8_m8192,dsv3_fp8_m1,dsv3_fp8_m128,"
    "mixtral_w4a16t_m1,mixtral_w4a16t_m4,mixtral_w4a16t_m16,mixtral_w4a16t_m64,"
    "mixtral_bf16_m1,mixtral_bf16_m16,mixtral_bf16_m256,"
    "qwen3_bf16_m1,qwen3_bf16_m64,qwen3_bf16_m1024,qwen3_bf16_m8192,tiny_bf16_m64,"
    + ",".join(f"refsweep_bf16_m{m}" for m in (1, 4, 17, 64, 1024, 2048, 4096)))
# secondaries that also get a CPU-oracle baseline (the north-star points and
# the other decode sizes the CPU finishes within its budget)
CPU_SECONDARY = ("dsv3_fp8_m4096", "dsv3_fp8_m1", "dsv3_fp8_m128", "mixtral_w4a16t_m1",
                 "mixtral_w4a16t_m4", "mixtral_w4a16t_m16")
STAGED_PATH_NOTE = ("staged path: the stage-level C ABI (align, [quant x], GEMM1, [quant act], GEMM2 "
                    "into fp32 planes, moe_sum), each timed with HIP events; the fused call runs the "
                    "same GEMM kernels but on fp8 prefill quantizes the activation in the GEMM1 "
                    "epilogue, writes bf16 GEMM2 rows when unsplit, and at M=1 (bf16, tiled int4) "
                    "takes single-token kernels -- so these stages do not add up to ms")


def _wt_codes():
    from flaggems_sglang import _lib

    return {"bf16": _lib.W_BF16, "fp8": _lib.W_FP8, "int4": _lib.W_INT4, "int4t": _lib.W_INT4_TILED,
            "mxfp4": _lib.W_MXFP4, "mxfp4t": _lib.W_MXFP4_TILED}


def _gen_weights(E, R, C, gen, dev, wtype, chunk=8):
    """N(0, 0.02) weights [E, R, C], quantized per wtype; generated a few
    experts at a time so the bf16 staging copy stays small."""
    import torch

    from flaggems_sglang import quant as Q

    outs = []
    for e0 in range(0, E, chunk):
        e1 = min(E, e0 + chunk)
        w = (torch.randn(e1 - e0, R, C, device=dev, generator=gen) * 0.02).to(torch.bfloat16)
        if wtype == "bf16":
            outs.append((w,))
        elif wtype == "fp8":
            outs.append(Q.quantize_fp8_block(w))
        elif wtype in ("mxfp4", "mxfp4t"):
            outs.append(Q.quantize_mxfp4(w))
        else:
            outs.append(Q.quantize_int4_group(w))
        del w
    if wtype in ("int4", "int4t"):
        # scales / zeros are [E, G, R]: concatenate along experts as well
        q, sc, z = (torch.cat([o[i] for o in outs]) for i in range(3))
        return (Q.tile_int4(q) if wtype == "int4t" else q), sc, z
    res = tuple(torch.cat([o[i] for o in outs]) for i in range(len(outs[0])))
    if wtype == "mxfp4t":
        res = (Q.tile_mxfp4(res[0]),) + res[1:]
    return res


def make_problem(name, seed=0):
    import torch

    import flaggems_sglang

    M, K, N, E, k, wtype, routing = WORKLOADS[name]
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(seed + M + K + N + E + k)
    x = torch.randn(M, K, device=dev, generator=gen).to(torch.bfloat16)
    w13 = _gen_weights(E, 2 * N, K, gen, dev, wtype)
    w2 = _gen_weights(E, K, N, gen, dev, wtype)
    logits = torch.randn(M, E, device=dev, generator=gen)
    if routing == "grouped":
        tw, ti = flaggems_sglang.grouped_topk(logits, k, 8, 4)
    else:
        if routing == "softmax_bias":
            logits = logits + torch.randn(E, device=dev, generator=gen)[None] * 0.5
        tw, ti = flaggems_sglang.topk_softmax(logits, k)
    kw = {}
    if wtype == "fp8":
        kw = dict(use_fp8_w8a8=True, w1_scale=w13[1], w2_scale=w2[1], block_shape=[128, 128])
    elif wtype in ("int4", "int4t"):
        kw = dict(use_int4_w4a16=True, w1_scale=w13[1], w2_scale=w2[1], w1_zp=w13[2], w2_zp=w2[2])
    elif wtype in ("mxfp4", "mxfp4t"):
        kw = dict(use_mxfp4_w4a16=True, w1_scale=w13[1], w2_scale=w2[1])
    return dict(name=name, M=M, K=K, N=N, E=E, k=k, wtype=wtype, x=x, w13=w13[0], w2=w2[0],
                tw=tw, ti=ti, kw=kw)


def flops(p):
    return 6.0 * p["M"] * p["k"] * p["K"] * p["N"]


def weight_bytes_touched(p):
    """Bytes of the experts the routing actually hits (+ scales / zeros)."""
    import torch

    hit = torch.bincount(p["ti"].flatten().long(), minlength=p["E"]).gt(0).sum().item()
    K, N = p["K"], p["N"]
    if p["wtype"] == "bf16":
        per = 3 * K * N * 2
    elif p["wtype"] == "fp8":
        per = 3 * K * N + 4 * (2 * N // 128) * (K // 128) + 4 * (K // 128) * (N // 128)
    elif p["wtype"] in ("mxfp4", "mxfp4t"):
        per = 3 * K * N // 2 + 3 * K * N // 32
    else:  # int4, row-major or tiled
        per = 3 * K * N // 2 + 2 * (K // 128) * 2 * N + (K // 128) * N + 2 * (N // 128) * K + (N // 128) * K // 2
    return hit, hit * per


def run_op(p, path=0):
    import flaggems_sglang

    return flaggems_sglang.fused_experts(p["x"], p["w13"], p["w2"], p["tw"], p["ti"], path=path, **p["kw"])


def time_op(p, steps, warmup, path=0):
    import torch

    for _ in range(warmup):
        run_op(p, path)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        run_op(p, path)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def time_op_graph(p, steps, min_bytes=2e9):
    """Device time of one call for small (decode) batches: L calls, each on its
    own copy of the weights (as the L MoE layers of a model; total above the
    256 MB last-level cache so no call finds its weights cached), captured in
    one HIP graph and replayed; time per call = replay time / L."""
    import torch

    tens = [p["w13"], p["w2"]] + [v for v in p["kw"].values() if torch.is_tensor(v)]
    wtot = sum(t.numel() * t.element_size() for t in tens)
    n_layers = min(64, max(1, int(min_bytes // max(wtot, 1)) + 1))
    layers = [p]
    for _ in range(n_layers - 1):
        q = dict(p)
        q["w13"] = p["w13"].clone()
        q["w2"] = p["w2"].clone()
        q["kw"] = {k: (v.clone() if torch.is_tensor(v) else v) for k, v in p["kw"].items()}
        layers.append(q)
    for q in layers:
        run_op(q)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run_op(p)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            outs = [run_op(q) for q in layers]
    torch.cuda.synchronize()
    ref = run_op(p)
    for _ in range(2):
        g.replay()
    torch.cuda.synchronize()
    if not all(torch.equal(o, ref) for o in outs):
        raise RuntimeError(f"{p['name']}: graph replay differs from the eager call")
    reps = max(3, steps // n_layers)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) * 1e-3 / reps / n_layers
    del g, outs, layers
    return t, n_layers


def stage_times(p, reps=10):
    """Per-stage device time (ms) through the stage-level C ABI (align, quant,
    GEMM1, quant, GEMM2, moe_sum), from HIP events recorded on the launch
    stream around each call.  The fused call runs the same GEMM kernels but
    folds two steps: on the fp8 prefill path the GEMM1 epilogue quantizes the
    activation (no separate quant_act pass), and without split-K its GEMM2
    rows are bf16 (halving the moe_sum read)."""
    import torch

    from flaggems_sglang import _lib
    from flaggems_sglang.ops import fused_moe as F

    L = _lib.lib()
    M, K, N, E, k = p["M"], p["K"], p["N"], p["E"], p["k"]
    wt = _wt_codes()[p["wtype"]]
    bm = L.fmoe_choose_block_m(wt, M, k, E, 0)
    kw = p["kw"]
    s13, s2 = kw.get("w1_scale"), kw.get("w2_scale")
    z13, z2 = kw.get("w1_zp"), kw.get("w2_zp")
    st = torch.cuda.current_stream().cuda_stream
    names = ["align", "quant_x", "gemm1", "quant_act", "gemm2", "moe_sum"]
    acc = {n: 0.0 for n in names}
    slots = M * k
    act = torch.empty(slots, N, dtype=torch.bfloat16, device="cuda")
    out = torch.empty(M, K, dtype=torch.bfloat16, device="cuda")
    for it in range(reps + 2):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(names) + 1)]
        # keep the GPU busy while the host enqueues the stages, so the events
        # bracket device time only (not host launch gaps)
        torch.cuda._sleep(4_000_000)
        ev[0].record()
        a = F._align(p["tw"], p["ti"], E, bm, False)
        r = _lib.Routing(a.topk_indx.data_ptr(), a.gate_indx.data_ptr(), a.gate_scal.data_ptr(),
                         a.offs_raw.data_ptr(), a.offs_pad.data_ptr(), a.tile_map.data_ptr(), a.n_tiles.data_ptr(), M, k, E,
                         bm, L.fmoe_max_tiles(slots, E))
        ev[1].record()
        xa, xs = p["x"], None
        if wt == _lib.W_FP8 and bm != 16:
            xa, xs = F.per_token_group_quant_fp8(p["x"])
        ev[2].record()
        _lib.check(L.fmoe_gemm1(wt, xa.data_ptr(), _lib.ptr(xs), p["w13"].data_ptr(), _lib.ptr(s13),
                                _lib.ptr(z13), K, N, ctypes.byref(r), 0, act.data_ptr(), 0, st), "gemm1")
        ev[3].record()
        aa, as_ = act, None
        if wt == _lib.W_FP8 and bm != 16:
            aa, as_ = F.per_token_group_quant_fp8(act)
        ev[4].record()
        splits = L.fmoe_gemm2_splits(wt, K, N, ctypes.byref(r), 0)
        y = torch.empty(splits, slots, K, dtype=torch.float32, device="cuda")
        _lib.check(L.fmoe_gemm2(wt, aa.data_ptr(), _lib.ptr(as_), p["w2"].data_ptr(), _lib.ptr(s2),
                                _lib.ptr(z2), K, N, ctypes.byref(r), 1, y.data_ptr(), splits, 0, st), "gemm2")
        ev[5].record()
        _lib.check(L.fmoe_moe_sum(y.data_ptr(), splits, a.gate_indx.data_ptr(), M, k, K, 1.0,
                                  out.data_ptr(), st), "moe_sum")
        ev[6].record()
        torch.cuda.synchronize()
        if it >= 2:
            for i, n in enumerate(names):
                acc[n] += ev[i].elapsed_time(ev[i + 1]) / reps
    if not (wt == _lib.W_FP8 and bm != 16):  # no separate quant passes ran
        del acc["quant_x"], acc["quant_act"]
    acc["block_m"] = bm
    return acc


def host_cores():
    """Cores this process may run on: the CPU affinity set, capped by a
    cgroup CPU quota when one is set (a GPU box grants each GPU a share of
    the host's cores)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            quota, period = f.read().split()[:2]
        if quota != "max":
            n = min(n, max(1, -(-int(quota) // int(period))))
    except (OSError, ValueError):
        pass
    return n


def _untile_4bit(t):
    """One expert of the tiled 4-bit layout [R/16, C/128, 1024] (byte
    16*(16*g + r) + i of block (b, c) = byte 64*c + 16*g + i of row 16*b + r)
    back to row-major [R, C/2]."""
    nb, nc, _ = t.shape
    return t.view(nb, nc, 4, 16, 16).permute(0, 3, 1, 2, 4).reshape(nb * 16, nc * 64)


class _HostExperts:
    """Per-expert host copies of a device weight tensor, made before the
    timed region (the oracle then indexes it like the tensor)."""

    def __init__(self, t, experts):
        self.shape = t.shape
        self.d = {e: t[e].cpu() for e in experts}

    def __getitem__(self, e):
        return self.d[e]


def cpu_baseline(p, budget_s=10.0):
    """The CPU oracle (fp32 torch restatement of the reference path, on all
    cores this process may use) on the first S tokens of the same problem, S
    sized to about budget_s seconds; the whole problem repeated when it fits.
    fp8 / int4 weights are dequantized one expert at a time inside the
    oracle, as a CPU implementation of those formats must (the DeepSeek-V3
    layer is 45 GB in fp32)."""
    import torch

    from oracle import fused_moe_oracle as O

    torch.set_num_threads(host_cores())
    x = p["x"].cpu()
    tw = p["tw"].cpu()
    ti = p["ti"].cpu()
    kw = p["kw"]
    if p["wtype"] == "bf16":
        w13, w2 = p["w13"].cpu(), p["w2"].cpu()
        fn = lambda S: O.fused_experts(x[:S], w13, w2, tw[:S], ti[:S])  # noqa: E731
    else:
        hit = sorted(set(ti.flatten().tolist()))
        hx = {n: _HostExperts(t, hit) for n, t in
              (("q1", p["w13"]), ("q2", p["w2"]), ("s1", kw["w1_scale"]), ("s2", kw["w2_scale"]))}
        if p["wtype"] == "fp8":
            fn = lambda S: O.fused_experts_fp8(x[:S], hx["q1"], hx["s1"], hx["q2"], hx["s2"],  # noqa: E731
                                               tw[:S], ti[:S])
        elif p["wtype"] in ("int4", "int4t"):
            if p["wtype"] == "int4t":  # the oracle reads the row-major packing
                hx["q1"].d = {e: _untile_4bit(v) for e, v in hx["q1"].d.items()}
                hx["q2"].d = {e: _untile_4bit(v) for e, v in hx["q2"].d.items()}
            z1, z2 = _HostExperts(kw["w1_zp"], hit), _HostExperts(kw["w2_zp"], hit)
            fn = lambda S: O.fused_experts_w4a16(x[:S], hx["q1"], hx["s1"], z1, hx["q2"],  # noqa: E731
                                                 hx["s2"], z2, tw[:S], ti[:S])
        else:
            return None

    def run(S):
        t0 = time.perf_counter()
        fn(S)
        return time.perf_counter() - t0

    S = min(p["M"], 64)
    t = run(S)
    while t < budget_s / 2 and S < p["M"]:
        S = int(min(p["M"], max(2 * S, S * budget_s / max(t, 1e-3))))
        t = run(S)
    # the whole workload fits the budget: repeat it and report the mean
    times = [t]
    while sum(times) < budget_s:
        times.append(run(S))
    t = sum(times) / len(times)
    f = 6.0 * S * p["k"] * p["K"] * p["N"]
    res = {"value": round(f / t / 1e12, 4), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
           "kind": "port",
           "sample": f"first {S} of {p['M']} tokens x {len(times)} runs, oracle/fused_moe_oracle.py "
                     f"({'fused_experts' if p['wtype'] == 'bf16' else 'fused_experts_' + p['wtype'].rstrip('t')}"
                     f", fp32 torch on CPU, per-expert weight upcast / dequantization included), "
                     f"{sum(times):.1f} s in total, mean {t:.3f} s per run"}
    if S == p["M"]:
        res["ms"] = round(t * 1e3, 2)
    return res


def _load_traffic(name):
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(name)
    except (OSError, ValueError):
        return None


def measure(name, steps, warmup, stages=True):
    import torch

    from flaggems_sglang import _lib

    p = make_problem(name)
    wt = _wt_codes()[p["wtype"]]
    decode = _lib.lib().fmoe_choose_block_m(wt, p["M"], p["k"], p["E"], 0) == 16
    timing = "wall clock per call, synchronous launches"
    if decode:
        for _ in range(warmup):
            run_op(p)
        t, n_layers = time_op_graph(p, steps)
        timing = f"HIP graph of {n_layers} calls on distinct weight copies, per call"
    else:
        t = time_op(p, steps, warmup)
    if stages:
        stages = stage_times(p)
    else:  # profiling the fused path alone: no staged-path launches in the trace
        stages = {"block_m": _lib.lib().fmoe_choose_block_m(wt, p["M"], p["k"], p["E"], 0)}
    f = flops(p)
    hit, wbytes = weight_bytes_touched(p)
    io_bytes = p["M"] * p["K"] * (2 if p["wtype"] != "fp8" else 1) + p["M"] * p["K"] * 2
    res = dict(p=p, t=t, stages=stages, flops=f, experts_hit=hit, bytes=wbytes + io_bytes,
               timing=timing)
    torch.cuda.synchronize()
    return res


def roofline_gemm1(res):
    """GEMM1+SiLU: algorithmic FLOPs 4*M*k*K*N per launch (bound mfma), or for
    decode the bytes of the touched w13 weights + x (bound hbm)."""
    p = res["p"]
    if "gemm1" not in res["stages"]:
        return None
    t = res["stages"]["gemm1"] * 1e-3
    decode = res["stages"]["block_m"] == 16
    if decode:
        hit = res["experts_hit"]
        K, N = p["K"], p["N"]
        if p["wtype"] in ("int4", "int4t"):
            wb = 2 * N * K // 2 + 2 * (K // 128) * 2 * N + (K // 128) * N
        elif p["wtype"] in ("mxfp4", "mxfp4t"):
            wb = 2 * N * K // 2 + 2 * N * K // 32
        elif p["wtype"] == "fp8":
            wb = 2 * N * K + 4 * (2 * N // 128) * (K // 128)
        else:
            wb = 2 * N * K * 2
        by = hit * wb + p["M"] * K * 2
        ach = by / t / 1e9
        return {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK["hbm_gbs"], "unit": "GB/s",
                "frac": round(ach / PEAK["hbm_gbs"], 4), "kernel": "gemm_decode_kernel<GEMM1+SiLU>",
                "algorithmic_bytes": by, "avg_ms": round(res["stages"]["gemm1"], 4)}
    fl = 4.0 * p["M"] * p["k"] * p["K"] * p["N"]
    ach = fl / t / 1e12
    peak = PEAK["fp8" if p["wtype"] == "fp8" else "bf16"]
    return {"bound": "mfma", "achieved": round(ach, 1), "peak": peak, "unit": "TFLOP/s",
            "frac": round(ach / peak, 4), "kernel": "gemm_prefill_kernel<GEMM1+SiLU>",
            "algorithmic_flops": fl, "avg_ms": round(res["stages"]["gemm1"], 4)}


def secondary_entry(res):
    p = res["p"]
    t = res["t"]
    tf = res["flops"] / t / 1e12
    gbs = res["bytes"] / t / 1e9
    e = {"workload": p["name"], "ms": round(t * 1e3, 4), "TFLOP/s": round(tf, 1),
         "GB/s": round(gbs, 1), "experts_hit": res["experts_hit"],
         "staged_path_ms": {k: round(v, 4) for k, v in res["stages"].items() if k != "block_m"},
         "block_m": res["stages"]["block_m"], "timing": res["timing"]}
    if res["stages"]["block_m"] == 16:
        e["frac_hbm_peak"] = round(gbs / PEAK["hbm_gbs"], 4)
    else:
        peak = PEAK["fp8" if p["wtype"] == "fp8" else "bf16"]
        ai = res["flops"] / res["bytes"]
        cap = min(peak, ai * PEAK["hbm_gbs"] / 1e3)
        e["frac_mfma_peak"] = round(tf / peak, 4)
        e["frac_of_min_peak_ai_bw"] = round(tf / cap, 4)
    return e


def measure_repack(reps=10):
    """Load-time int4 checkpoint repack (AWQ and GPTQ v2) of the Mixtral w13
    shape [8, 2*14336 rows, K=4096], group 128: HBM bytes read + written per
    call over the call's time."""
    import torch

    from flaggems_sglang import formats as F

    E, K, N, g = 8, 4096, 2 * 14336, 128
    dev = "cuda"
    gen = torch.Generator(device=dev).manual_seed(5)
    out = {}
    for fmt in ("awq", "gptq_v2"):
        shape = (E, K, N // 8) if fmt == "awq" else (E, K // 8, N)
        qw = torch.randint(-2**31, 2**31 - 1, shape, dtype=torch.int32, device=dev, generator=gen)
        qz = torch.randint(-2**31, 2**31 - 1, (E, K // g, N // 8), dtype=torch.int32, device=dev, generator=gen)
        sc = torch.rand(E, K // g, N, device=dev, generator=gen).to(torch.float16)
        fn = (lambda: F.repack_awq_moe(qw, qz, sc)) if fmt == "awq" else \
            (lambda: F.repack_gptq_moe(qw, qz, sc, checkpoint_format="gptq_v2"))
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) / reps / 1e3
        nbytes = 2 * (qw.numel() * 4 + qz.numel() * 4 + sc.numel() * 2)
        out[fmt] = {"ms": round(t * 1e3, 4), "GB/s": round(nbytes / t / 1e9, 1),
                    "frac_hbm_peak": round(nbytes / t / 1e9 / PEAK["hbm_gbs"], 4),
                    "bytes": nbytes}
        del qw, qz, sc
        torch.cuda.empty_cache()
    return {"workload": "int4 checkpoint repack, Mixtral w13 [8, 28672, 4096], group 128", **out}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="mixtral_bf16_m4096", choices=sorted(WORKLOADS))
    ap.add_argument("--secondary", default=DEFAULT_SECONDARY,
                    help="comma list of extra workloads reported in 'secondary' ('' for none)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-stages", action="store_true",
                    help="skip the staged-path stage timing (and the roofline computed from it), so a "
                         "kernel trace holds the fused path's launches only")
    ap.add_argument("--copy-calib", action="store_true",
                    help="also run a plain 1 GiB device copy 5x (reference kernel for scaling "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the fused-MoE kernels on one "
              "device's share); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(2)

    head = measure(args.workload, args.steps, args.warmup, stages=not args.no_stages)
    p = head["p"]
    line = {
        "metric": "fused_moe TFLOP/s & % MFMA peak (prefill); HBM GB/s % peak (decode), 1 GPU",
        "value": round(head["flops"] / head["t"] / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["t"] * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"bf16": "bf16", "fp8": "fp8-e4m3 (fp32 acc)", "int4": "int4 w / bf16 a",
                  "int4t": "int4 w (tiled) / bf16 a", "mxfp4": "mxfp4 w / bf16 a",
                  "mxfp4t": "mxfp4 w (tiled) / bf16 a"}[p["wtype"]],
        "data": "synthetic: x~N(0,1), weights~N(0,0.02) random-init, router logits~N(0,1)",
        "config": {"workload": p["name"], "M": p["M"], "K": p["K"], "N": p["N"], "E": p["E"],
                   "top_k": p["k"], "weights": p["wtype"], "global_batch": p["M"],
                   "parallelism": "single GPU"},
        "staged_path_ms": {k: round(v, 4) for k, v in head["stages"].items() if k != "block_m"},
        "staged_path": STAGED_PATH_NOTE,
    }
    rl = roofline_gemm1(head)
    tr = _load_traffic(p["name"])
    if rl is not None:
        rl["traffic"] = None if tr is None else tr["bytes"]
        if tr is not None:
            rl["traffic_detail"] = {k: tr[k] for k in ("read_bytes", "write_bytes", "calibration", "source")}
    line["roofline"] = rl
    sec = []
    for name in [s for s in args.secondary.split(",") if s and s != args.workload]:
        r = measure(name, max(5, args.steps // 2), args.warmup, stages=not args.no_stages)
        e = secondary_entry(r)
        if name in CPU_SECONDARY and not args.no_cpu:
            e["cpu_baseline"] = cpu_baseline(r["p"], budget_s=6.0)
        sec.append(e)
        del r
        torch.cuda.empty_cache()
    line["secondary"] = sec
    line["repack"] = measure_repack()
    line["cpu_baseline"] = None if args.no_cpu else cpu_baseline(p)
    if args.copy_calib:
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
