#!/usr/bin/env python
"""Benchmark of the MoE feed-forward block on one MI355X.

Workload: the Qwen3-30B-A3B-shape MoE layer,
forward + backward, T = 8192 tokens (batch 4 x seq 2048), hidden 2048,
128 experts, top-8, moe_intermediate 768, SwiGLU, bf16 activations and
weights with an fp32 router. One step = router + experts forward and the full
backward (upstream grad N(0,1)), inputs resident in HBM.

Prints one JSON line: tokens/s (whole job), expert-GEMM TFLOP/s and its
fraction of the bf16 dense MFMA peak, per-stage HIP-event timings, the
roofline of the dominant kernel, HBM GB/s of the row-movement kernels, the
reference's own torch GPU path (F.grouped_mm) timed on the same GPU and
inputs, the MoE half-block with and without the fused RMSNorm / residual add
(``neighbours``), the other BASELINE.json configurations' steps (``decode``:
config 5, ``config4``: skewed routing, ``config3``: the Qwen3-235B-A22B layer;
``config2_fp16``: config 2 with fp16 tensors, router weight included, on the fp16 MFMAs; ``ep8_share``:
one GPU's share at EP=8), the forward expert GEMMs against
hipBLASLt's batched product on equal experts (``vendor_gemm``), and a CPU
baseline (the restated reference CPU path) timed on this host.

Two timed regions of --steps steps each: the first, bracketed by two events,
gives ms_per_step and tokens/s; the second records an event pair around each
stage (kernel) for the per-kernel durations.
"""

from __future__ import annotations

import argparse
import contextlib
import dataclasses
import json
import math
import os
import platform
import statistics
import sys
import time

PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16 MFMA (256 CU x 2.4 GHz x 4096 FLOP/clk)
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
METRIC = "MoE layer fwd+bwd tokens/s & TFLOP/s (% bf16 MFMA peak), Qwen3-30B-A3B shape"


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=2, help="workload id (BASELINE.json configs, 1-based)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-reference-gpu", action="store_true",
                    help="skip timing the reference's own torch path (F.grouped_mm) on this GPU")
    ap.add_argument("--no-neighbours", action="store_true",
                    help="skip timing the MoE half-block with and without the fused RMSNorm / residual add")
    ap.add_argument("--neighbours-only", action="store_true",
                    help="time only the MoE half-block in the trainer's regime and print its JSON object "
                         "(for profiling that regime on its own)")
    ap.add_argument("--cpu-tokens", type=int, default=256,
                    help="tokens of the CPU-baseline sample (0: the full workload)")
    ap.add_argument("--no-decode", action="store_true",
                    help="skip the legs after the config-2 line: config 5 (decode, 64 tokens), the EP=8 share, "
                         "config 4 (skewed routing) and config 3 (the Qwen3-235B-A22B layer)")
    ap.add_argument("--copy-mib", type=int, default=256,
                    help="size of the device-to-device copy timed as the measured HBM reference (0: skip)")
    return ap.parse_args()


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(cfg, tokens: int | None, iters: int = 3):
    """The reference CPU path (router + per-expert loop, autograd backward), restated in oracle/.

    One warm-up step, then ``iters`` timed runs (each of as many steps as
    fill about a second); the median per step is reported. The
    sample is the first ``tokens`` tokens' worth of the workload (a fresh
    seeded draw of that size, same layer shape)."""
    import torch

    from oracle import moe_oracle as O
    from pluggy_amd.workloads import make_inputs

    T = cfg.tokens if not tokens else min(tokens, cfg.tokens)
    inp = make_inputs(cfg, tokens=T)
    H = cfg.hidden

    def step():
        x = inp["x"].reshape(1, T, H).detach().requires_grad_(cfg.backward)
        params = [inp["router_weight"], inp["gate_up_proj"], inp["down_proj"]]
        wr, gu, dn = (p.detach().requires_grad_(cfg.backward) for p in params)
        y, _ = O.sparse_mlp_forward(x, wr, gu, dn, cfg.top_k, cfg.norm_topk_prob, logit_bias=inp.get("logit_bias"))
        if cfg.backward:
            y.reshape(T, H).backward(inp["grad_out"])

    t0 = time.perf_counter()
    step()  # warm-up
    # a timed run repeats the step until it lasts about a second (config 1's
    # forward takes milliseconds), so the median is not timer noise
    reps = max(1, math.ceil(1.0 / max(time.perf_counter() - t0, 1e-3)))
    times = []
    for _ in range(iters):
        t0 = time.perf_counter()
        for _ in range(reps):
            step()
        times.append((time.perf_counter() - t0) / reps)
    dt = statistics.median(times)
    return {
        "value": round(T / dt, 2),
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{'fwd+bwd' if cfg.backward else 'fwd'} steps of the restated reference CPU path (fp32 router + "
                   f"per-expert loop, moe.py:38-65, torch autograd) at T={T} of the {cfg.name} layer, {cfg.dtype}: "
                   f"1 warm-up + {iters} timed runs of {reps} step(s), median {dt:.4g} s per step "
                   f"(runs {', '.join(f'{t:.4g}' for t in times)} s)"),
        "cpu_model": cpu_model(),
        "os_cpu_count": os.cpu_count(),
        "torch": torch.__version__,
    }


def reference_gpu(cfg, inp, steps: int, warmup: int, dev):
    """The reference's own GPU path, timed on this GPU on the same inputs.

    ``Qwen3MoeSparseMLP.forward`` as the trainer runs it, under
    ``torch.autocast(cuda, bf16)`` (trainer.py:469): router ``F.linear`` (bf16
    logits), fp32 softmax, ``torch.topk``, renormalise, cast (qwen3_moe.py:
    168-178); experts by the sorted/grouped path (moe.py:68-124: stable
    argsort, bincount + cumsum offsets, two ``F.grouped_mm``, SwiGLU, weighted
    ``index_add_``); torch autograd for the backward. Restated with torch ops
    for this comparison only; the product never runs it.
    """
    import torch
    import torch.nn.functional as F

    T, H, E, K = cfg.tokens, cfg.hidden, cfg.experts, cfg.top_k
    x, gout, bias = inp["x"], inp.get("grad_out"), inp.get("logit_bias")
    params = [inp[n].detach().clone().requires_grad_(cfg.backward)
              for n in ("router_weight", "gate_up_proj", "down_proj")]
    token_idx = torch.arange(T, device=dev).unsqueeze(1).expand(T, K).reshape(-1)

    def step():
        for p in params:
            p.grad = None
        wr, gu, dn = params
        xg = x.detach().requires_grad_(cfg.backward)
        dt = xg.dtype
        with torch.autocast("cuda", dtype=torch.bfloat16):
            logits = F.linear(xg, wr)
            if bias is not None:
                logits = logits + bias
            probs = F.softmax(logits, dim=-1, dtype=torch.float32)
            top_w, top_i = torch.topk(probs, K, dim=-1)
            if cfg.norm_topk_prob:
                top_w = top_w / top_w.sum(dim=-1, keepdim=True)
            top_w = top_w.to(dt)
            expert_idx = top_i.reshape(-1)
            order = torch.argsort(expert_idx, stable=True)
            sorted_token = token_idx[order]
            sorted_w = top_w.reshape(-1)[order]
            offs = torch.cumsum(torch.bincount(expert_idx[order], minlength=E), dim=0).to(torch.int32)
            gate_up = F.grouped_mm(xg[sorted_token], gu.to(dt).transpose(-2, -1), offs=offs)
            gate, up = gate_up.chunk(2, dim=-1)
            y = F.grouped_mm(F.silu(gate) * up, dn.to(dt).transpose(-2, -1), offs=offs)
            y = y * sorted_w.unsqueeze(1).to(dt)
            out = torch.zeros(T, H, device=dev, dtype=dt).index_add_(0, sorted_token, y)
        if cfg.backward:
            out.backward(gout)

    for _ in range(warmup):
        step()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(steps):
        step()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    return {"value": round(T / (ms * 1e-3), 1), "unit": "tokens/s", "ms_per_step": round(ms, 4), "steps": steps,
            "path": "reference Qwen3MoeSparseMLP under bf16 autocast: F.linear router + torch.topk, "
                    "F.grouped_mm experts (moe.py:68-124), torch autograd backward; same inputs"}


def neighbours(cfg, inp, steps: int, warmup: int, dev):
    """The MoE half of a transformer block, ``x + SparseMLP(RMSNorm(x))``
    (qwen3_moe.py:281), fwd+bwd as the trainer runs it: fp32 residual stream and
    fp32 master weights under bf16 autocast (trainer.py:469). Unfused = torch's
    RMSNorm, the drop-in MLP and torch's add; fused = ``moe_sublayer`` (norm in
    the row kernel that feeds the router, residual add in the combine, their
    backward in the dispatch backward)."""
    import torch

    import pluggy_amd

    T, H, E, K, I = cfg.tokens, cfg.hidden, cfg.experts, cfg.top_k, cfg.inter
    B = cfg.batch
    norm = torch.nn.RMSNorm(H).to(dev)
    mlp = pluggy_amd.Qwen3MoeSparseMLP(H, I, E, K, cfg.norm_topk_prob).to(dev)
    with torch.no_grad():
        mlp.router.weight.copy_(inp["router_weight"])
        mlp.experts.gate_up_proj.copy_(inp["gate_up_proj"].float())
        mlp.experts.down_proj.copy_(inp["down_proj"].float())
    x = inp["x"].float().reshape(B, T // B, H)
    gout = inp["grad_out"].float().reshape(B, T // B, H)
    params = list(norm.parameters()) + list(mlp.parameters())

    def step(fused):
        for p in params:
            p.grad = None
        xg = x.detach().requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            out = pluggy_amd.moe_sublayer(xg, norm, mlp) if fused else xg + mlp(norm(xg))
        out.backward(gout)

    res = {}
    for name, fused, cached in (("unfused_ms", False, False), ("fused_ms", True, False),
                                ("fused_cached_ms", True, True)):
        ctx = pluggy_amd.weight_cast_cache() if cached else contextlib.nullcontext()
        with ctx:
            for _ in range(warmup):
                step(fused)
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            start.record()
            for _ in range(steps):
                step(fused)
            end.record()
            torch.cuda.synchronize()
        res[name] = round(start.elapsed_time(end) / steps, 4)
    res["saved_ms"] = round(res["unfused_ms"] - res["fused_ms"], 4)
    # fused_cached_ms: each step a micro-batch between optimizer steps, reusing the bf16 copies of
    # the fp32 masters (pluggy_amd.weight_cast_cache); the copy is made once per optimizer step,
    # cast_ms_per_copy is what that costs
    res["cast_ms_per_copy"] = round(res["fused_ms"] - res["fused_cached_ms"], 4)
    res["regime"] = "x + SparseMLP(RMSNorm(x)) fwd+bwd, fp32 residual stream and fp32 master weights, bf16 autocast"
    return res


def decode_leg(dev, steps: int = 50, warmup: int = 5):
    """Config 5: a 64-token forward of the config-2
    layer, where most experts get 0-4 rows and the expert weights stream from
    HBM. Reports ms per forward and the weight-stream GB/s of the two expert
    GEMMs (each hit expert's gate_up and down weights read once) against the
    HBM peak."""
    import torch

    import pluggy_amd
    from pluggy_amd.moe import stage_timer
    from pluggy_amd.workloads import CONFIGS, make_inputs

    cfg = CONFIGS[5]
    T, H, E, K, I = cfg.tokens, cfg.hidden, cfg.experts, cfg.top_k, cfg.inter
    inp = make_inputs(cfg, device=dev)
    mlp = pluggy_amd.Qwen3MoeSparseMLP(H, I, E, K, cfg.norm_topk_prob).to(dev)
    with torch.no_grad():
        mlp.router.weight.copy_(inp["router_weight"])
    mlp.experts.gate_up_proj.data = inp["gate_up_proj"]
    mlp.experts.down_proj.data = inp["down_proj"]
    x = inp["x"].reshape(1, T, H)
    with torch.no_grad():
        for _ in range(warmup):
            mlp(x)
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        for _ in range(steps):
            mlp(x)
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / steps
        with stage_timer() as timer:
            for _ in range(steps):
                mlp(x)
            torch.cuda.synchronize()
        # the same forward captured in a HIP graph and replayed (a serving loop's form)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            mlp(x)
        for _ in range(warmup):
            graph.replay()
        torch.cuda.synchronize()
        start.record()
        for _ in range(steps):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
        graph_ms = start.elapsed_time(end) / steps
        # one forward at a time, the host waiting for each (a decode loop's
        # latency, host launch work included): eager calls, then graph replays
        sync_ms = {}
        for name, fn in (("eager", lambda: mlp(x)), ("graph", graph.replay)):
            t0 = time.perf_counter()
            for _ in range(steps):
                fn()
                torch.cuda.synchronize()
            sync_ms[name] = (time.perf_counter() - t0) * 1e3 / steps
        del graph
    st = timer.summary()
    hit = int((mlp.router.last_stats.expert_counts > 0).sum().item())
    es = 2
    gu_b, dn_b = hit * 2 * I * H * es, hit * H * I * es
    gemm_ms = st["gate_up_fwd"]["mean_ms"] + st["down_fwd"]["mean_ms"]
    gbs = (gu_b + dn_b) / (gemm_ms * 1e-3) / 1e9
    return {"workload": f"{cfg.name} fwd (T={T}, layer as config 2)", "ms_per_forward": round(ms, 4),
            "graph_ms_per_forward": round(graph_ms, 4),
            "synced_ms_per_forward": {k: round(v, 4) for k, v in sync_ms.items()},
            "tokens/s": round(T / (ms * 1e-3), 1), "experts_hit": hit,
            "weight_bytes": gu_b + dn_b, "expert_gemms_ms": round(gemm_ms, 4),
            "weight_stream_GB/s": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4),
            "gate_up_fwd_GB/s": round(gu_b / (st["gate_up_fwd"]["mean_ms"] * 1e-3) / 1e9, 1),
            "down_fwd_GB/s": round(dn_b / (st["down_fwd"]["mean_ms"] * 1e-3) / 1e9, 1),
            "stages_ms": {n: round(v["mean_ms"], 4) for n, v in sorted(st.items(), key=lambda kv: -kv[1]["total_ms"])}}


def layer_leg(cfg_id: int, dev, steps: int, warmup: int, base_inp=None, base_ms=None, dtype=None):
    """Another BASELINE.json configuration's whole layer step (router, experts,
    and the backward for fwd+bwd configs), timed like the headline line: HIP
    events around `steps` steps after `warmup`. Config 4 reuses config 2's
    tensors (`base_inp`: the same seeded draws) with its Zipf logit bias and
    reports the routing's per-expert counts and its step time relative to
    config 2's (`base_ms`). `dtype`: the configuration with its activations and
    expert weights in that dtype instead (config 2 in fp16: the same draws
    rounded to fp16, the router weight included, as a module in fp16 holds
    them: the reference's F.linear takes fp16 input only beside an fp16
    weight)."""
    import dataclasses

    import torch

    import pluggy_amd
    from pluggy_amd.workloads import CONFIGS, make_inputs, zipf_logit_bias

    cfg = CONFIGS[cfg_id]
    if dtype is not None and dtype != cfg.dtype:
        cfg = dataclasses.replace(cfg, name=f"{cfg.name}-{str(dtype).split('.')[-1]}", dtype=dtype)
    T, H, E, K, I = cfg.tokens, cfg.hidden, cfg.experts, cfg.top_k, cfg.inter
    if base_inp is not None:
        inp = dict(base_inp)
        if cfg.skew:
            inp["logit_bias"] = zipf_logit_bias(E, cfg.skew).to(dev)
        for key in ("x", "gate_up_proj", "down_proj", "grad_out"):
            if key in inp:
                inp[key] = inp[key].to(cfg.dtype)
    else:
        inp = make_inputs(cfg, device=dev)
    mlp = pluggy_amd.Qwen3MoeSparseMLP(H, I, E, K, cfg.norm_topk_prob).to(dev)
    if cfg.dtype == torch.float16:
        mlp.router.to(torch.float16)
    with torch.no_grad():
        mlp.router.weight.copy_(inp["router_weight"])
    mlp.experts.gate_up_proj.data = inp["gate_up_proj"]
    mlp.experts.down_proj.data = inp["down_proj"]
    mlp.router.logit_bias = inp.get("logit_bias")
    x = inp["x"].reshape(cfg.batch, T // cfg.batch, H)
    gout = inp["grad_out"].reshape(x.shape) if cfg.backward else None

    def step():
        for p in mlp.parameters():
            p.grad = None
        xg = x.detach().requires_grad_(cfg.backward)
        out = mlp(xg)
        if cfg.backward:
            out.backward(gout)

    for _ in range(warmup):
        step()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(steps):
        step()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    tflops = cfg.gemm_flops() / (ms * 1e-3) / 1e12
    out = {"workload": f"{cfg.name} MoE layer {'fwd+bwd' if cfg.backward else 'fwd'} (T={T}, H={H}, E={E}, "
                       f"K={K}, I={I})",
           "ms_per_step": round(ms, 4), "tokens/s": round(T / (ms * 1e-3), 1), "steps": steps, "warmup": warmup,
           "TFLOP/s": round(tflops, 1), "mfma_frac": round(tflops / PEAK_BF16_TFLOPS, 4)}
    counts = mlp.router.last_stats.expert_counts
    if cfg.skew:
        out["expert_rows_min_max"] = [int(counts.min().item()), int(counts.max().item())]
    if base_ms:
        out["vs_config2_step"] = round(ms / base_ms, 3)
    out["dtype"] = str(cfg.dtype).split(".")[-1]
    del mlp, inp
    torch.cuda.empty_cache()
    return out


def vendor_gemm_leg(dev, launches: int = 20, warmup: int = 5):
    """The forward expert GEMMs against the vendor library on the problem it can
    run: 128 equal experts of 512 rows (config 2's shape with uniform routing),
    where the grouped product is a plain batched one. Ours: gate_up with the
    SwiGLU epilogue (it also writes the activation) and down, on the sorted rows;
    the library's: torch.bmm (hipBLASLt) on the same operands, the weights
    pre-transposed to contiguous (E, K, N) copies. The two alternate launch by
    launch, each timed with its own pair of HIP events, so that both see the
    same clock as the chip warms; the medians are reported."""
    import torch

    from pluggy_amd import ops

    E, R, H, I = 128, 512, 2048, 768
    g = torch.Generator().manual_seed(4)
    xp = torch.randn(E * R, H, generator=g).to(torch.bfloat16).to(dev)
    wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    wdn = (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    offs = (torch.arange(1, E + 1, dtype=torch.int32) * R).to(dev)
    wgu_t, wdn_t = wgu.transpose(1, 2).contiguous(), wdn.transpose(1, 2).contiguous()
    _, mid = ops.gate_up_swiglu(xp, wgu, offs)

    def timed_pair(fa, fb):
        """Median ms of fa and of fb, launched alternately."""
        for _ in range(warmup):
            fa()
            fb()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(3 * launches)]
        torch.cuda.synchronize()
        for i in range(launches):
            ev[3 * i].record()
            fa()
            ev[3 * i + 1].record()
            fb()
            ev[3 * i + 2].record()
        torch.cuda.synchronize()
        ta = sorted(ev[3 * i].elapsed_time(ev[3 * i + 1]) for i in range(launches))
        tb = sorted(ev[3 * i + 1].elapsed_time(ev[3 * i + 2]) for i in range(launches))
        return ta[launches // 2], tb[launches // 2]

    xp3, mid3 = xp.view(E, R, H), mid.view(E, R, I)
    out = {"problem": f"{E} experts x {R} rows, H={H}, I={I}, bf16", "launches": launches,
           "timing": "alternating launches, median of each"}
    for name, ours, lib, flop in (
            ("gate_up", lambda: ops.gate_up_swiglu(xp, wgu, offs), lambda: torch.bmm(xp3, wgu_t),
             2.0 * E * R * H * 2 * I),
            ("down", lambda: ops.down_proj(mid, wdn, offs), lambda: torch.bmm(mid3, wdn_t), 2.0 * E * R * I * H)):
        t_ours, t_lib = timed_pair(ours, lib)
        out[name] = {"ours_us": round(t_ours * 1e3, 1), "ours_TFLOP/s": round(flop / (t_ours * 1e-3) / 1e12, 1),
                     "hipblaslt_bmm_us": round(t_lib * 1e3, 1),
                     "hipblaslt_TFLOP/s": round(flop / (t_lib * 1e-3) / 1e12, 1),
                     "speedup": round(t_lib / t_ours, 3)}
    del xp, wgu, wdn, wgu_t, wdn_t, mid
    torch.cuda.empty_cache()
    return out


def ep_share_leg(dev, ep: int = 8, steps: int = 20, warmup: int = 5):
    """One GPU's share of config 2 under expert parallelism over `ep` GPUs
    (design only in this build: no all-to-all runs). GPU 0 owns experts
    [0, E/ep); it receives the config-2 pairs routed to them (their token rows,
    one row per pair, with the routing weight) and runs the expert FFN forward
    and backward on those rows alone: `moe_expert_ffn` with K = 1 over E/ep
    experts, the same kernels at the per-GPU shape. The ids are the router's,
    so the operator's host-side id check (one synchronising read per call,
    which the reference's F.one_hot / bincount also make) is timed apart and
    left out of `ms_per_step`."""
    import torch

    import pluggy_amd
    import pluggy_amd.moe as pmoe_moe
    from pluggy_amd.workloads import CONFIGS, make_inputs

    cfg = CONFIGS[2]
    T, H, E, K, I = cfg.tokens, cfg.hidden, cfg.experts, cfg.top_k, cfg.inter
    El = E // ep
    inp = make_inputs(cfg, device=dev)
    _, tw, ti = pluggy_amd.router_topk(inp["x"], inp["router_weight"], K)
    sel = ti.reshape(-1) < El
    tok = torch.arange(T, device=dev).repeat_interleave(K)[sel]
    rows = inp["x"][tok].contiguous()
    idx = ti.reshape(-1)[sel].reshape(-1, 1).contiguous()
    w = tw.reshape(-1)[sel].reshape(-1, 1).contiguous()
    gu = inp["gate_up_proj"][:El].clone().requires_grad_(True)
    dn = inp["down_proj"][:El].clone().requires_grad_(True)
    g = torch.randn(rows.shape, generator=torch.Generator().manual_seed(3)).to(rows.dtype).to(dev)
    P = rows.shape[0]

    def step():
        x = rows.detach().requires_grad_(True)
        y = pluggy_amd.moe_expert_ffn(x, idx, w, gu, dn)
        y.backward(g)
        gu.grad = dn.grad = None

    def timed():
        for _ in range(warmup):
            step()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        for _ in range(steps):
            step()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps

    ms_checked = timed()
    prev, pmoe_moe.VALIDATE_EXPERT_IDS = pmoe_moe.VALIDATE_EXPERT_IDS, False
    try:
        ms = timed()
    finally:
        pmoe_moe.VALIDATE_EXPERT_IDS = prev
    flops = 3.0 * (2.0 * P * H * 2 * I + 2.0 * P * I * H)
    tf = flops / (ms * 1e-3) / 1e12
    return {"workload": f"expert FFN fwd+bwd of one GPU's share at EP={ep} of {cfg.name}: {El} experts, "
                        f"{P} received rows (all-to-all not run)",
            "experts": El, "rows": P, "ms_per_step": round(ms, 4), "TFLOP/s": round(tf, 1),
            "mfma_frac": round(tf / PEAK_BF16_TFLOPS, 4), "ms_per_step_with_id_check": round(ms_checked, 4)}


def copy_bandwidth(mib: int, dev, reps: int = 5):
    """HIP-event time of a plain device-to-device copy of `mib` MiB (read + write counted).

    Runs after the timed region. Its rocprofv3 FETCH_SIZE / WRITE_SIZE readings
    calibrate the counters against a known byte count.
    """
    import torch

    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    dst.copy_(src)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        dst.copy_(src)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / reps
    return {"bytes_per_copy": n, "mean_ms": round(ms, 4), "GB/s": round(2 * n / (ms * 1e-3) / 1e9, 1)}


def profiled_traffic(workload: str) -> dict:
    """HBM bytes per launch of each kernel, from the committed rocprofv3 summary.

    ``profiles/traffic_<workload>.txt`` holds lines ``kernel <name> avg_us <t>
    hbm_bytes <b>`` computed from FETCH_SIZE / WRITE_SIZE passes (scaled by a
    copy kernel of known size). Missing file -> {} (traffic reported as null).
    """
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"traffic_{workload}.txt")
    out = {}
    try:
        with open(path) as f:
            for line in f:
                tok = line.split()
                if len(tok) >= 6 and tok[0] == "kernel" and tok[4] == "hbm_bytes":
                    out[tok[1]] = int(tok[5])
    except OSError:
        return out
    out["_source"] = os.path.relpath(path, os.path.dirname(os.path.abspath(__file__)))
    return out


GEMM_STAGES = ("gate_up_fwd", "down_fwd", "down_dgrad", "down_wgrad", "gate_up_dgrad", "gate_up_wgrad")


def main() -> int:
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE={world}). Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    import pluggy_amd
    from pluggy_amd.moe import stage_timer
    from pluggy_amd.workloads import CONFIGS, combine_bytes, make_inputs

    cfg = CONFIGS[args.config]
    assert torch.cuda.is_available(), "bench.py needs a ROCm GPU"
    dev = torch.device("cuda:0")
    T, H, E, K, I = cfg.tokens, cfg.hidden, cfg.experts, cfg.top_k, cfg.inter
    P = cfg.pairs
    inp = make_inputs(cfg, device=dev)
    mlp = pluggy_amd.Qwen3MoeSparseMLP(H, I, E, K, cfg.norm_topk_prob).to(dev)
    with torch.no_grad():
        mlp.router.weight.copy_(inp["router_weight"])
    mlp.experts.gate_up_proj.data = inp["gate_up_proj"]
    mlp.experts.down_proj.data = inp["down_proj"]
    if "logit_bias" in inp:
        mlp.router.logit_bias = inp["logit_bias"]
    B = cfg.batch
    if args.neighbours_only:
        assert cfg.backward and cfg.hidden <= 16384, "the half-block leg needs a fwd+bwd workload with H <= 16384"
        print(json.dumps({"workload": cfg.name, "neighbours": neighbours(cfg, inp, args.steps, args.warmup, dev)}),
              flush=True)
        return 0
    x = inp["x"].reshape(B, T // B, H)
    gout = inp.get("grad_out")
    gout = gout.reshape(B, T // B, H) if gout is not None else None

    def step():
        for p in mlp.parameters():
            p.grad = None
        xg = x.detach().requires_grad_(cfg.backward)
        out = mlp(xg)
        if cfg.backward:
            out.backward(gout)
        return out

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # Timed region 1: K whole steps, bracketed by two HIP events only (an event
    # record between kernels leaves a gap of ~10 us on the GPU, so per-stage
    # events would inflate the step time).
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        step()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(end) / args.steps
    # Timed region 2: K more steps with HIP events around every stage (each
    # kernel's duration on the stream it runs on) for the roofline and the
    # per-stage breakdown.
    with stage_timer() as timer:
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
    stages = timer.summary()

    traffic = profiled_traffic(cfg.name)
    gemm_flops = cfg.gemm_flops()
    tflops = gemm_flops / (ms * 1e-3) / 1e12
    es = cfg.dtype.itemsize
    # dominant kernel: the grouped-GEMM stage with the largest total time
    gemm = {n: s for n, s in stages.items() if n in GEMM_STAGES}
    dom = max(gemm, key=lambda n: gemm[n]["total_ms"])
    # algorithmic FLOPs and HBM bytes per launch of each expert GEMM: every
    # operand read once and every output written once; an expert's weights are
    # read only when it has rows (the last step's routing counts). The
    # token-major operands the GEMMs gather (hidden in gate_up fwd / wgrad, the
    # output gradient in down dgrad / wgrad) count once per token (T*H); each
    # gathered GEMM also reads its P sorted-row indices (and weights).
    active = int((mlp.router.last_stats.expert_counts > 0).sum().item())
    w_gu, w_dn = active * 2 * I * H * es, active * H * I * es
    tok = T * H * es
    gemm_work = {
        "gate_up_fwd": (2.0 * P * H * 2 * I, w_gu + tok + P * 8 + P * 2 * I * es + P * I * es),
        "down_fwd": (2.0 * P * I * H, w_dn + P * I * es + P * H * es),
        "down_dgrad": (2.0 * P * H * I, tok + P * 8 + w_dn + 2 * P * 2 * I * es + P * ((I + 63) // 64) * 4),
        "down_wgrad": (2.0 * P * H * I, tok + P * 4 + P * I * es + w_dn),
        "gate_up_dgrad": (2.0 * P * 2 * I * H, P * 2 * I * es + w_gu + P * H * es),
        "gate_up_wgrad": (2.0 * P * 2 * I * H, P * 2 * I * es + tok + P * 4 + w_gu),
    }
    dom_flops, dom_bytes = gemm_work[dom]
    dom_s = gemm[dom]["mean_ms"] * 1e-3
    dom_tflops, dom_gbs = dom_flops / dom_s / 1e12, dom_bytes / dom_s / 1e9
    # roofline: the bound is whichever peak gives the longer minimum time
    intensity = dom_flops / dom_bytes
    ridge = PEAK_BF16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)
    mfma_view = {"achieved": round(dom_tflops, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                 "frac": round(dom_tflops / PEAK_BF16_TFLOPS, 4)}
    hbm_view = {"achieved": round(dom_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(dom_gbs / PEAK_HBM_GBS, 4)}
    bound = "mfma" if intensity >= ridge else "hbm"
    hbm = {}
    for name, nbytes in (("combine", combine_bytes(cfg)),
                         # the block's backward hands the router's input gradient to
                         # the dispatch backward as its addend: one more (T, H) read
                         ("dispatch_bwd", P * H * es + P * 4 + 2 * T * H * es),
                         # x, W (fp32), fp32 logits out, top-k ids / weights out
                         ("router_fwd", T * H * es + E * H * 4 + T * E * 4 + T * K * (es + 8 + 4)),
                         # x, W, logits, ids, fp32 weights and their gradient in; dx, dW out
                         ("router_bwd", 2 * T * H * es + 2 * E * H * 4 + T * E * 4 + T * K * (8 + 4 + 4))):
        if name in stages:
            t_ms = stages[name]["mean_ms"]
            if name == "router_fwd" and "router_split" in stages:
                # the fp32 weight's bf16 pieces, made before the router op (its backward reuses them)
                t_ms += stages["router_split"]["mean_ms"]
            gbs = nbytes / (t_ms * 1e-3) / 1e9
            hbm[name] = {"bytes": nbytes, "mean_ms": round(t_ms, 4), "GB/s": round(gbs, 1),
                         "frac": round(gbs / PEAK_HBM_GBS, 4)}

    result = {
        "metric": METRIC,
        "value": round(T / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {torch.bfloat16: "bf16", torch.float16: "f16"}.get(cfg.dtype, "f32"),
        "data": "synthetic (seeded N(0,1) inputs and upstream grad, N(0,0.02) weights)",
        "config": {"workload": f"{cfg.name} MoE layer {'fwd+bwd' if cfg.backward else 'fwd'}", "tokens": T,
                   "batch": B, "seq_len": T // B, "hidden": H, "experts": E, "top_k": K, "moe_intermediate": I,
                   "router": "fp32", "parallelism": "single GPU"},
        "tflops": round(tflops, 2),
        "mfma_frac": round(tflops / PEAK_BF16_TFLOPS, 4),
        "gemm_gflop_per_step": round(gemm_flops / 1e9, 1),
        "wall_s": round(wall, 3),
        "roofline": {"kernel": dom, "bound": bound, **(mfma_view if bound == "mfma" else hbm_view),
                     "traffic": traffic.get(dom), "traffic_source": traffic.get("_source"),
                     "flop_per_launch": dom_flops, "bytes_per_launch": dom_bytes,
                     "intensity_flop_per_byte": round(intensity, 1), "ridge_flop_per_byte": round(ridge, 1),
                     "mfma_view": mfma_view, "hbm_view": hbm_view, "mean_ms": round(gemm[dom]["mean_ms"], 4)},
        # traffic_ratio: the profiled HBM bytes per launch (profiles/traffic_<workload>.txt) over the
        # algorithmic bytes above; above 1 means re-reads past L2 (and the Infinity Cache, which
        # FETCH_SIZE also counts)
        "gemm_stages": {n: {"TFLOP/s": round(f / (gemm[n]["mean_ms"] * 1e-3) / 1e12, 1),
                            "GB/s": round(b / (gemm[n]["mean_ms"] * 1e-3) / 1e9, 1),
                            "intensity": round(f / b, 1), "bytes_per_launch": b,
                            "traffic_ratio": round(traffic[n] / b, 3) if n in traffic else None}
                        for n, (f, b) in gemm_work.items() if n in gemm},
        "hbm": hbm,
        "stages_ms": {n: round(s["mean_ms"], 4) for n, s in sorted(stages.items(), key=lambda kv: -kv[1]["total_ms"])},
        "cpu_baseline": None,
    }
    if args.copy_mib > 0:
        result["copy_reference"] = copy_bandwidth(args.copy_mib, dev)
    if not args.no_neighbours and cfg.backward and cfg.hidden <= 16384:
        result["neighbours"] = neighbours(cfg, inp, min(args.steps, 10), 2, dev)
    if not args.no_reference_gpu:
        ref = reference_gpu(cfg, inp, min(args.steps, 10), 2, dev)
        ref["speedup"] = round(result["value"] / ref["value"], 2)
        result["reference_gpu"] = ref
    if not args.no_decode and args.config == 2:
        result["decode"] = decode_leg(dev)
        result["ep8_share"] = ep_share_leg(dev)
        result["config4"] = layer_leg(4, dev, args.steps, args.warmup, base_inp=inp, base_ms=ms)
        # the same layer with fp16 tensors (the fp16 MFMA path), against the bf16 step
        result["config2_fp16"] = layer_leg(2, dev, args.steps, args.warmup, base_inp=inp, base_ms=ms,
                                           dtype=torch.float16)
        result["config3"] = layer_leg(3, dev, min(args.steps, 10), 3)
        result["vendor_gemm"] = vendor_gemm_leg(dev)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(cfg, args.cpu_tokens)
        if args.config == 2:
            # the reference's own CPU-runnable case: fp32 forward, whole workload;
            # and the decode forward, whole workload
            result["cpu_baseline_config1"] = cpu_baseline(CONFIGS[1], 0)
            result["cpu_baseline_config5"] = cpu_baseline(CONFIGS[5], 0)
            # the skewed routing and the headline layer in fp32, on 128-token samples
            result["cpu_baseline_config4"] = cpu_baseline(CONFIGS[4], 128)
            result["cpu_baseline_config2_fp32"] = cpu_baseline(
                dataclasses.replace(CONFIGS[2], dtype=torch.float32, name="qwen3-30b-a3b-fp32"), 128)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
