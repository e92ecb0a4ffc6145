#!/usr/bin/env python3
"""Throughput of the MI355X token-sampling path (TVdxSampler on the GPU).

A step is one batched sampling call over B resident rows of V fp32 logits:
repetition penalty (in place) + top-K select + softmax / Top-P / draw, all in
libvdxsampler.so's HIP kernels.  Prints ONE JSON line (rank 0).

Default workload (the metric's B=64, top-k 64 / top-p 0.95 configuration):
  penalised batch, B=64, V=262144, logits 3*N(0,1) + 6 at 32 hot ids per
  row, a 256-id history per row (half from the hot ids, half uniform), RP 1.1
  (window 256), T 0.8, top-k 64, top-p 0.95, the sampler's own per-row RNG.

Inputs are resident in HBM before timing.  Logits cycle through a pool of
buffers totalling >= 2 GiB so no step is served from the 256 MiB MALL; the
pool is restored from a pristine copy (outside the timed region) before each
measured phase, so the in-place penalty (applied again each time a buffer is
reused, as the reference does on its input) stays far from overflow.  The timed loop is K
steps bracketed by torch.cuda.synchronize(); by default the steps are issued
from a captured hipGraph (one node per pool buffer), the way a serving loop
issues them; --eager issues every call from Python instead.

roofline: each step is one kernel launch; HIP events recorded on the launch
stream around the timed region give its mean duration; achieved = algorithmic
bytes per launch (logit bytes read once, B*V*4) / that duration.  traffic =
HBM bytes per launch from rocprofv3 FETCH_SIZE + WRITE_SIZE, each scaled by
the same counter's reading for a 1 GiB device copy (bench.py --traffic-from
turns the two counter CSVs into profiles/traffic_<workload>.json).
cpu_baseline: the oracle (oracle/vdx_oracle.c, a C restatement of
TVdxSampler.Process, gcc -O2) on one host core over a bounded sample;
cpu_baseline_all_cores: the same split over the job's host threads.
reference_readback: the step's device-to-host logits copy that the
reference pipeline pays before its host sampler (pageable and pinned).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

METRIC = "rows/sec sampled (B=64, V=262144, topk64/topp0.95); % of HBM peak"
MIN_TIMED = 128          # fewest steps in a timed region
NORTH_STAR = "topk_b256"  # B=256 top-k 64 / top-p 0.95: the >= 60% of HBM target
EXTRA = ("topk128_b64", "topk_only_b64")
HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, AMD published
POOL_BYTES = 2 << 30

WORKLOADS = {
    "penalised_b64": dict(
        rows=64, vocab=262144, hist=256,
        cfg=dict(Temperature=0.8, TopK=64, TopP=0.95, RepeatPenalty=1.1, RepeatWindow=256, Seed=3003),
        desc="penalised B=64 V=262144 3N(0,1)+6@32 ids, 256-id history, RP 1.1, T 0.8, top-k 64, top-p 0.95"),
    "topk_b256": dict(
        rows=256, vocab=262144, hist=0,
        cfg=dict(Temperature=1.0, TopK=64, TopP=0.95, Seed=3006),
        desc="B=256 V=262144 3N(0,1)+8@16 ids, T 1.0, top-k 64, top-p 0.95"),
    "full_b256": dict(
        rows=256, vocab=262144, hist=0,
        cfg=dict(Temperature=0.7, TopK=0, TopP=0.9, Seed=3004),
        desc="full-vocab B=256 V=262144 Zipf logits, T 0.7, top-k 0 (TopP ignored as in the reference)"),
    "topk128_b64": dict(
        rows=64, vocab=262144, hist=0,
        cfg=dict(Temperature=1.0, TopK=128, TopP=0.95, Seed=3011),
        desc="B=64 V=262144 3N(0,1)+8@16 ids, T 1.0, top-k 128, top-p 0.95 (large-K kernel)"),
    "topk_only_b64": dict(
        rows=64, vocab=262144, hist=0,
        cfg=dict(Temperature=1.0, TopK=64, TopP=1.0, Seed=3012),
        desc="B=64 V=262144 3N(0,1)+8@16 ids, T 1.0, top-k 64, top-p 1 (draw in slot order: exact path)"),
    "greedy_b64": dict(
        rows=64, vocab=262144, hist=0, cfg=dict(Temperature=0.0, Seed=3002),
        desc="greedy argmax B=64 V=262144, 4 tied maxima/row"),
    "single_row": dict(
        rows=1, vocab=262144, hist=0, cfg=dict(Temperature=1.0, TopK=64, TopP=0.95, Seed=3001),
        desc="B=1 V=262144 fp32 3*N(0,1)+8 at 16 ids, T 1.0, top-k 64, top-p 0.95"),
    "mixed_rows_b64": dict(
        rows=64, vocab=262144, hist=256,
        cfg=dict(Temperature=0.8, TopK=64, TopP=0.95, RepeatPenalty=1.1, RepeatWindow=256, Seed=3007),
        row_cfgs=[dict(Temperature=0.8, TopK=64, TopP=0.95, RepeatPenalty=1.1, RepeatWindow=256, Seed=3007),
                  dict(Temperature=0.0, RepeatPenalty=1.2, RepeatWindow=64, Seed=3008),
                  dict(Temperature=0.7, TopK=40, TopP=0.9, MinP=0.05, RepeatPenalty=1.3,
                       RepeatWindow=128, Seed=3009),
                  dict(Temperature=1.0, TopK=0, RepeatPenalty=1.1, RepeatWindow=256, Seed=3010)],
        desc="per-row configs B=64 V=262144, rows cycle top-k 64/top-p 0.95, greedy, "
             "top-k 40/min-p 0.05, full softmax; all penalised"),
}
# the kernel(s) of one step: K > 64 runs as a stream launch and a per-row finish launch
DOMINANT_KERNEL = {"penalised_b64": "k_topk_vec", "topk_b256": "k_topk_vec",
                   "topk128_b64": "k_topk_big_stream_vec+k_topk_big_finish_vec", "topk_only_b64": "k_topk_vec+k_topk_exact_vec",
                   "full_b256": "k_full<true,false>", "greedy_b64": "k_greedy<true>",
                   "single_row": "k_topk_vec", "mixed_rows_b64": "k_topk_vec"}


def make_inputs(name, seed=1000):
    w = WORKLOADS[name]
    rng = np.random.default_rng(seed)
    B, V = w["rows"], w["vocab"]
    hist = None
    if name == "full_b256":
        L = np.empty((B, V), dtype=np.float32)
        lr = np.log(np.arange(1, V + 1, dtype=np.float64))
        for r in range(B):
            L[r] = (-1.1 * lr[rng.permutation(V)] + 0.5 * rng.standard_normal(V)).astype(np.float32)
        return L, hist
    L = (3.0 * rng.standard_normal((B, V))).astype(np.float32)
    if name in ("penalised_b64", "mixed_rows_b64"):
        hist = np.zeros((B, w["hist"]), dtype=np.int32)
        for r in range(B):
            hot = rng.choice(V, 32, replace=False)
            L[r, hot] += np.float32(6.0)
            h = np.concatenate([rng.choice(hot, w["hist"] // 2), rng.integers(0, V, w["hist"] // 2)])
            rng.shuffle(h)
            hist[r] = h
    elif name == "greedy_b64":
        for r in range(B):
            L[r, rng.choice(V, 4, replace=False)] = L[r].max() + 1.0
    else:
        for r in range(B):
            L[r, rng.choice(V, 16, replace=False)] += np.float32(8.0)
    return L, hist


def configure(s, w):
    c = s.DefaultConfig()
    for k, v in w["cfg"].items():
        setattr(c, k, v)
    s.SetConfig(c)
    rc = w.get("row_cfgs")
    for r in range(w["rows"] if rc else 0):
        c = s.DefaultConfig()
        for k, v in rc[r % len(rc)].items():
            setattr(c, k, v)
        s.SetRowConfig(r, c)


def cpu_model() -> str:
    """The host CPU's model name (Linux /proc/cpuinfo), or '' where unreadable."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def host_threads() -> int:
    """Host threads for the all-cores baseline: the job's CPU share where the
    environment states it (OMP_NUM_THREADS), else every core."""
    n = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, int(n) if n.isdigit() else (os.cpu_count() or 1))


def cpu_baseline(name, L, hist, seconds, threads=1):
    """The oracle on the host: with threads=1 rows are processed serially, as
    the reference's Process does; with more, the rows are split over that many
    POSIX threads (one independent sampler each).  A bounded sample of
    ~`seconds` of wall-clock work."""
    from oracle import vdx_oracle as O

    w = WORKLOADS[name]
    c = w["cfg"]
    cfg = O.make_config(temperature=c.get("Temperature", 0.0), top_k=c.get("TopK", 0),
                        top_p=c.get("TopP", 1.0), min_p=c.get("MinP", 0.0),
                        repeat_penalty=c.get("RepeatPenalty", 1.0),
                        repeat_window=c.get("RepeatWindow", 64))
    B = L.shape[0]
    u = (np.random.default_rng(7).integers(0, 2**24, B) / 2**24).astype(np.float32)
    rows_done, busy, passes = 0, 0.0, 0
    while busy < seconds:
        X = L.copy()
        t0 = time.perf_counter()
        O.process_batch(X, cfg, u, hist=hist, threads=threads)
        busy += time.perf_counter() - t0
        rows_done += B
        passes += 1
    return dict(value=rows_done / busy, unit="rows/s", cores=threads, kind="port", cpu=cpu_model(),
                sample=f"{passes} passes x {B} rows of the same workload ({busy:.1f} s), "
                       f"oracle/vdx_oracle.c gcc -O2, {threads} thread{'s' if threads > 1 else ''}")


def readback_cost(rows, vocab, reps=50):
    """What the reference pipeline pays before its host sampler runs: one
    device-to-host copy of the step's logits (rows x vocab fp32,
    Inference.pas:332-334) into pageable and into pinned host memory."""
    import torch

    dev = torch.device("cuda:0")
    src = torch.empty(rows, vocab, dtype=torch.float32, device=dev).normal_()
    out = {"bytes": rows * vocab * 4}
    for kind in ("pageable", "pinned"):
        dst = torch.empty(rows, vocab, dtype=torch.float32, pin_memory=(kind == "pinned"))
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        for _ in range(reps):
            dst.copy_(src)
        torch.cuda.synchronize(dev)
        us = 1e6 * (time.perf_counter() - t0) / reps
        out[f"{kind}_us"] = us
        out[f"{kind}_GBs"] = out["bytes"] / (us * 1e-6) / 1e9
    return out


def run_gpu(name, steps, warmup, eager, check=False):
    import torch

    from vindexllm_amd import TVdxSampler

    w = WORKLOADS[name]
    B, V = w["rows"], w["vocab"]
    L, hist = make_inputs(name)
    dev = torch.device("cuda:0")
    step_bytes = B * V * 4
    P = max(2, math.ceil(POOL_BYTES / step_bytes))
    pristine = torch.from_numpy(L).to(dev)
    pool = [pristine.clone() for _ in range(P)]
    tok = torch.empty(B, dtype=torch.int32, device=dev)
    s = TVdxSampler(0, B)
    configure(s, w)
    if hist is not None:
        for r in range(B):
            s.set_history(r, hist[r][:max(s.GetRowConfig(r).RepeatWindow, 0)])
    stream = torch.cuda.current_stream(dev)
    for i in range(max(warmup, 1)):
        s.process_device(pool[i % P], tokens=tok, stream=stream)
    torch.cuda.synchronize()

    def restore():
        for b in pool:
            b.copy_(pristine)
        torch.cuda.synchronize()

    # The timed region runs exactly `steps` steps: steps // P replays of a
    # graph over the whole pool, then one replay of a graph over the first
    # steps % P buffers.
    graph = rest = None
    if not eager:
        cs = torch.cuda.Stream(dev)
        cs.wait_stream(stream)
        with torch.cuda.stream(cs):
            s.process_device(pool[0], tokens=tok, stream=cs)  # workspace already sized
        torch.cuda.synchronize()

        def capture(n):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=cs):
                for i in range(n):
                    s.process_device(pool[i], tokens=tok, stream=cs)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            return g

        graph = capture(P)
        if steps % P:
            rest = capture(steps % P)

    restore()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    if graph is not None:
        for _ in range(steps // P):
            graph.replay()
        if rest is not None:
            rest.replay()
    else:
        for i in range(steps):
            s.process_device(pool[i % P], tokens=tok, stream=stream)
    ev1.record(stream)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    # Every step of these workloads is ONE kernel launch (penalty fused into the
    # top-K kernel, no separate max pass), so the events bracketing the timed
    # region on the launch stream give the kernel's mean duration (plus the
    # inter-node gap of the graph, which makes the figure conservative).
    kernel_ms = ev0.elapsed_time(ev1) / steps

    # which path the rows took (one call on restored inputs)
    restore()
    fl = torch.zeros(B, dtype=torch.int32, device=dev)
    s.process_device(pool[0], tokens=tok, flags=fl, stream=stream)
    torch.cuda.synchronize()
    flags = fl.cpu().numpy()
    s.Free()
    out = dict(steps=steps, elapsed=elapsed, rows=B, vocab=V, step_bytes=step_bytes, pool=P,
               kernel_ms=kernel_ms,
               launch="hipGraph" if graph is not None else "eager",
               fast_frac=float(((flags & 0x2) != 0).mean()),
               replay_frac=float(((flags & 0x4) != 0).mean()))
    if check:
        out["parity"] = parity_check(name, L, hist)
    return out


def parity_check(name, L, hist, seed=4242):
    """One sampling call on the workload's own pristine inputs with injected
    per-row uniforms, outside any timed region, checked row by row against
    the oracle (oracle/vdx_oracle.c): greedy and top-K tokens, top-K index
    sets and penalised logits must be bit-exact; a full-softmax token may
    differ only within 1e-6*S of a CDF boundary (counted)."""
    import torch

    from oracle import vdx_oracle as O
    from vindexllm_amd import TVdxSampler

    w = WORKLOADS[name]
    B, V = L.shape
    dev = torch.device("cuda:0")
    u = (np.random.default_rng(seed).integers(0, 2**24, B) / 2**24).astype(np.float32)
    d = torch.from_numpy(L).to(dev)
    s = TVdxSampler(0, B)
    configure(s, w)
    if hist is not None:
        for r in range(B):
            s.set_history(r, hist[r][:max(s.GetRowConfig(r).RepeatWindow, 0)])
    Kmax = max([w["cfg"].get("TopK", 0)] + [c.get("TopK", 0) for c in w.get("row_cfgs", [])] + [1])
    ti = torch.full((B, Kmax), -1, dtype=torch.int32, device=dev)
    fl = torch.zeros(B, dtype=torch.int32, device=dev)
    tok = s.process_device(d, uniforms=torch.from_numpy(u).to(dev), topk_idx=ti, flags=fl)
    torch.cuda.synchronize()
    tok, ti, fl, after = tok.cpu().numpy(), ti.cpu().numpy(), fl.cpu().numpy(), d.cpu().numpy()
    s.Free()
    rc = w.get("row_cfgs")
    mism = bnd = set_mism = logit_mism = 0
    t0 = time.perf_counter()
    for r in range(B):
        c = rc[r % len(rc)] if rc else w["cfg"]
        cfg = O.make_config(temperature=c.get("Temperature", 0.0), top_k=c.get("TopK", 0),
                            top_p=c.get("TopP", 1.0), min_p=c.get("MinP", 0.0),
                            repeat_penalty=c.get("RepeatPenalty", 1.0), repeat_window=c.get("RepeatWindow", 64))
        row = L[r].copy()
        h = hist[r][:max(c.get("RepeatWindow", 64), 0)] if hist is not None else None
        want, tr = O.process_row(row, cfg, float(u[r]), hist=h, trace=True)
        if not np.array_equal(row.view(np.uint32), after[r].view(np.uint32)):
            logit_mism += 1
        if tr.path == O.PATH_TOPK:
            K = tr.k
            order = sorted(range(K), key=lambda k: (-float(np.float32(tr.slot_val[k])), tr.slot_idx[k]))
            if ti[r][:K].tolist() != [tr.slot_idx[k] for k in order]:
                set_mism += 1
        if tok[r] != want:
            dist = (min(tr.target - tr.cdf_lo, tr.cdf_hi - tr.target) / tr.sum_final
                    if tr.sum_final > 0 and np.isfinite(tr.sum_final) else np.inf)
            if tr.path == O.PATH_FULL and dist < 1e-6:
                bnd += 1
            else:
                mism += 1
    return {"rows": B, "token_mismatches": mism, "boundary_draws": bnd, "topk_set_mismatches": set_mism,
            "penalised_logit_mismatches": logit_mism,
            "rows_fast_path": int(((fl & 0x2) != 0).sum()), "rows_replay_path": int(((fl & 0x4) != 0).sum()),
            "oracle_s": round(time.perf_counter() - t0, 3),
            "bar": "tokens/top-K sets/penalised logits bit-exact; full-path draws within 1e-6*S of a "
                   "boundary counted"}


LMHEAD_V, LMHEAD_D = 262144, 2560  # Gemma-3-4B tied lm_head (token_embd.weight)
LMHEAD_CHAIN = 16  # calls per captured graph for the steady-state figures
VALU_FP32_PEAK_TFLOPS = 157.3      # MI355X published FP32 vector peak (packed FMA)


LMHEAD_FORMATS = {"q4_0": (2, 18), "q8_0": (8, 34), "f16": (1, 64)}  # GGML type id, bytes per 32


def run_lmhead(B, steps, warmup, fmt="q4_0", norm=False, packed=True, eager=False):
    """lm_head + sampling with the logits kept in HBM (RunUnembedding followed
    by Process, Inference.pas:327-339): the lm_head of 262144 x 2560 in `fmt`
    (Q4_0: nibbles uniform 0..15; Q8_0: int8 uniform; fp16 scales
    |N(0, 0.02)|; F16: N(0, 0.05)), optionally after the output RMSNorm, over
    B hidden rows N(0, 1), then top-k 64 / top-p 0.95 / T 1.0.  With `packed`
    the weights are first repacked once (lmhead_pack, outside the timed
    region) and read in that layout.  Times the whole call and the lm_head
    alone (norm included), each from a captured hipGraph (or issued one by
    one with `eager`, for counter collection)."""
    import torch

    from vindexllm_amd import VDX_LMHEAD_PACKED, TVdxSampler, lmhead, lmhead_pack

    V, D = LMHEAD_V, LMHEAD_D
    wtype, bb = LMHEAD_FORMATS[fmt]
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(1005)
    nb = D // 32
    if fmt == "f16":
        w = (torch.randn(V, D, device=dev, generator=g) * 0.05).half().view(torch.uint8)
    else:
        w = torch.randint(0, 256, (V, nb, bb), dtype=torch.uint8, device=dev, generator=g)
        d = (torch.randn(V, nb, device=dev, generator=g) * 0.02).abs().half()
        w[:, :, 0:2] = d.view(torch.uint8).view(V, nb, 2)
    w = w.reshape(-1)
    if packed:
        w = lmhead_pack(w, wtype, D, V)
        wtype = wtype | VDX_LMHEAD_PACKED
        torch.cuda.synchronize()
    hidden = torch.randn(B, D, device=dev, generator=g)
    nw = (1.0 + 0.1 * torch.randn(D, device=dev, generator=g)) if norm else None
    logits = torch.empty(B, V, dtype=torch.float32, device=dev)
    scratch = torch.empty(16 * D, dtype=torch.float32, device=dev)
    tok = torch.empty(B, dtype=torch.int32, device=dev)
    s = TVdxSampler(0, B)
    c = s.DefaultConfig()
    c.Temperature, c.TopK, c.TopP, c.Seed = 1.0, 64, 0.95, 3005
    s.SetConfig(c)
    cs = torch.cuda.Stream(dev)
    cs.wait_stream(torch.cuda.current_stream(dev))

    def both():
        s.lmhead_device(w, wtype, hidden, V, norm_weight=nw, logits=logits, tokens=tok, stream=cs)

    def head():
        lmhead(w, wtype, hidden, V, norm_weight=nw, logits=logits, scratch=scratch, stream=cs)

    res = {}
    for tag, fn in (("call", both), ("lmhead", head)):
        with torch.cuda.stream(cs):
            for _ in range(max(warmup, 1)):
                fn()
        torch.cuda.synchronize()
        if eager:
            rs = cs
            run = fn
        else:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=cs):
                fn()
            graph.replay()
            torch.cuda.synchronize()
            # replay() launches on torch's current stream: the events go there
            rs = torch.cuda.current_stream(dev)
            run = graph.replay
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(rs)
        for _ in range(steps):
            run()
        e1.record(rs)
        torch.cuda.synchronize()
        res[tag] = dict(wall_us=1e6 * (time.perf_counter() - t0) / steps,
                        event_us=1e3 * e0.elapsed_time(e1) / steps)
        if not eager:
            # the same call CHAIN times over in one graph: the steady-state
            # cost of a call inside a larger captured step (a decode loop's
            # whole forward is one graph), without one graph launch per call
            chain = torch.cuda.CUDAGraph()
            with torch.cuda.graph(chain, stream=cs):
                for _ in range(LMHEAD_CHAIN):
                    fn()
            chain.replay()
            torch.cuda.synchronize()
            reps = max(1, steps // LMHEAD_CHAIN)
            e0.record(rs)
            for _ in range(reps):
                chain.replay()
            e1.record(rs)
            torch.cuda.synchronize()
            res[tag]["chain_event_us"] = 1e3 * e0.elapsed_time(e1) / (reps * LMHEAD_CHAIN)
    s.Free()
    head_us = res["lmhead"]["event_us"]
    weight_bytes = V * nb * bb
    alg_bytes = weight_bytes + B * D * 4
    flops = 2.0 * V * D * B
    out = {"rows_per_s": B / (res["call"]["wall_us"] * 1e-6),
           "us_per_step": res["call"]["wall_us"],
           "call_event_us": res["call"]["event_us"],
           "call_chain_event_us": res["call"].get("chain_event_us"),
           "lmhead_kernel_us": head_us,
           "lmhead_chain_event_us": res["lmhead"].get("chain_event_us"),
           "lmhead_gbs": alg_bytes / (head_us * 1e-6) / 1e9,
           "lmhead_hbm_frac": alg_bytes / (head_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
           "lmhead_tflops": flops / (head_us * 1e-6) / 1e12,
           "lmhead_valu_frac": flops / (head_us * 1e-6) / 1e12 / VALU_FP32_PEAK_TFLOPS,
           "bound": "hbm" if B == 1 else "valu",
           "desc": f"{fmt.upper()} lm_head {V}x{D}{' + output RMSNorm' if norm else ''} + top-k 64/top-p 0.95, "
                   f"B={B} hidden rows N(0,1), weights {'packed (lmhead_pack)' if packed else 'in the GGUF layout'}"}
    return out


def run_host_process(steps=300, warmup=20, penalised=False):
    """The host entry point as the reference calls it (Process on one host row,
    Inference.pas:327-339): each call uploads the 1 MiB row over PCIe, samples
    it (B=1 top-k 64 / top-p 0.95 / T 1.0) and returns the token to the host.
    penalised: RP 1.1 over a 64-id history as well, so each call also writes
    the penalised history positions back into the caller's row (the row is
    penalised again on every call, as the reference would).
    The PCIe-inclusive rate, reported beside `value`, never as it."""
    import torch

    from vindexllm_amd import TVdxSampler

    w = WORKLOADS["single_row"]
    L, _ = make_inputs("single_row")
    row = np.ascontiguousarray(L[0])
    s = TVdxSampler(0, 1)
    configure(s, w)
    if penalised:
        c = s.GetConfig()
        c.RepeatPenalty, c.RepeatWindow = 1.1, 64
        s.SetConfig(c)
        for t in np.random.default_rng(11).integers(0, row.size, 64):
            s.AddToHistory(int(t))
    for _ in range(warmup):
        s.Process(row)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        s.Process(row)
    dt = (time.perf_counter() - t0) / steps
    s.Free()
    return {"rows_per_s": 1.0 / dt, "us_per_call": 1e6 * dt,
            "desc": "vdx_sampler_process on a pageable host row: B=1 V=262144, 1 MiB upload + sampling + token "
                    "download per call, top-k 64 / top-p 0.95 / T 1.0"
                    + (", RP 1.1 over 64 history ids (penalised positions written back)" if penalised else "")}


def copy_calibration(nbytes=1 << 30, reps=5):
    """Device-to-device copies of a known size, for scaling rocprofv3's
    FETCH_SIZE / WRITE_SIZE counters (run under --pmc)."""
    import torch

    a = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda:0").fill_(1.0)
    b = torch.empty_like(a)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()


PMC_COMMAND = ("timeout -s KILL 60 rocprofv3 --pmc {counter} -f csv -d gpurun_out/pmc_{tag}_{workload} -o {tag} -- "
               "python -u bench.py --workload {workload} --eager --steps 20 --warmup 3 --no-cpu "
               "--no-check --no-north-star --copy-calibration")


def _kernel_base(name):
    name = name.strip()
    if name.startswith("void "):
        name = name[5:]
    name = name.split("(")[0].strip().replace(", ", ",")  # template arguments as in DOMINANT_KERNEL
    return name[5:] if name.startswith("vdx::") else name


def _counter_rows(path, counter):
    import csv

    with open(path, newline="") as f:
        return [(_kernel_base(r["Kernel_Name"]), float(r["Counter_Value"]))
                for r in csv.DictReader(f) if r["Counter_Name"] == counter]


def traffic_from(workload, fetch_csv, write_csv, calib_bytes=1 << 30):
    """Scale FETCH_SIZE / WRITE_SIZE (KiB per dispatch) of the step's kernel
    by what the same counters read for a device copy of calib_bytes, and write
    profiles/traffic_<workload>.json.  A step of several launches ("a+b")
    adds each kernel's median dispatch."""
    kernel = DOMINANT_KERNEL[workload]
    names = kernel.split("+")
    out = {"workload": workload, "kernel": kernel, "calibration_copy_bytes": calib_bytes,
           "algorithmic_bytes_per_launch": WORKLOADS[workload]["rows"] * WORKLOADS[workload]["vocab"] * 4}
    total = 0.0
    for counter, path, tag in (("FETCH_SIZE", fetch_csv, "fetch"), ("WRITE_SIZE", write_csv, "write")):
        rows = _counter_rows(path, counter)
        copies = [v for k, v in rows if "copyBuffer" in k]
        meds, ndisp = [], []
        for name in names:
            kern = sorted(v for k, v in rows if k == name)
            if not kern:
                raise SystemExit(f"{path}: no {counter} rows for {name}")
            meds.append(kern[len(kern) // 2])
            ndisp.append(len(kern))
        if not copies:
            raise SystemExit(f"{path}: no {counter} rows for the calibration copy")
        calib = max(copies)  # the calib_bytes copies are the largest copy dispatches
        factor = calib_bytes / (calib * 1024.0)
        med = sum(meds)
        out[f"{tag}_kib_per_dispatch_raw"] = med if len(meds) == 1 else meds
        out[f"{tag}_dispatches"] = ndisp[0] if len(ndisp) == 1 else ndisp
        out[f"{tag}_calibration_kib_raw"] = calib
        out[f"{tag}_scale"] = factor
        out[f"{tag}_bytes_per_launch"] = med * 1024.0 * factor
        out[f"{tag}_command"] = PMC_COMMAND.format(counter=counter, tag=tag, workload=workload)
        total += med * 1024.0 * factor
    out["traffic_bytes_per_launch"] = total
    out["traffic_over_algorithmic"] = total / out["algorithmic_bytes_per_launch"]
    os.makedirs(os.path.join(ROOT, "profiles"), exist_ok=True)
    dst = os.path.join(ROOT, "profiles", f"traffic_{workload}.json")
    with open(dst, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(json.dumps(out))


def read_traffic(name):
    p = os.path.join(ROOT, "profiles", f"traffic_{name}.json")
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f).get("traffic_bytes_per_launch")
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--workload", default="penalised_b64", choices=sorted(WORKLOADS))
    ap.add_argument("--eager", action="store_true", help="issue every step from Python")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-check", action="store_true", help="skip the oracle parity check of the inputs")
    ap.add_argument("--no-north-star", action="store_true", help="skip the B=256 north-star workload")
    ap.add_argument("--others", action="store_true", help="also measure the other workloads")
    ap.add_argument("--copy-calibration", action="store_true")
    ap.add_argument("--lmhead", type=int, metavar="B",
                    help="only the lm_head + sampling workload at B hidden rows (one JSON line)")
    ap.add_argument("--lmhead-format", default="q4_0", choices=sorted(LMHEAD_FORMATS))
    ap.add_argument("--lmhead-gguf-layout", action="store_true",
                    help="read the weights in their GGUF layout instead of the packed one")
    ap.add_argument("--lmhead-norm", action="store_true", help="fuse the output RMSNorm")
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="no GPU: turn two rocprofv3 --pmc counter CSVs into profiles/traffic_<workload>.json")
    a = ap.parse_args()
    if a.traffic_from:
        traffic_from(a.workload, *a.traffic_from)
        return
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: measures one GPU; the sampling path has no multi-GPU "
              "collective (rows shard with zero exchange), so --gpus must be 1", file=sys.stderr)
        sys.exit(3)

    if a.lmhead:
        print(json.dumps(run_lmhead(a.lmhead, min(a.steps, 500), min(a.warmup, 20), fmt=a.lmhead_format,
                                    norm=a.lmhead_norm, packed=not a.lmhead_gguf_layout, eager=a.eager)),
              flush=True)
        if a.copy_calibration:
            copy_calibration()
        return
    # at least MIN_TIMED steps are timed (a few hundred microseconds of work
    # is too short a region to be stable); "steps" reports the count timed
    steps = max(a.steps, MIN_TIMED)
    r = run_gpu(a.workload, steps, a.warmup, a.eager, check=not a.no_check)
    rows_s = r["rows"] * r["steps"] / r["elapsed"]
    ms_step = 1e3 * r["elapsed"] / r["steps"]
    achieved = r["step_bytes"] / (r["kernel_ms"] * 1e-3) / 1e9
    out = {
        "metric": METRIC,
        "value": rows_s,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": r["steps"],
        "steps_requested": a.steps,
        "warmup": a.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": WORKLOADS[a.workload]["desc"], "rows": r["rows"], "vocab": r["vocab"],
                   "launch": r["launch"], "pool_buffers": r["pool"],
                   "us_per_row": 1e3 * ms_step / r["rows"],
                   "hbm_frac_step": (r["step_bytes"] / (ms_step * 1e-3) / 1e9) / HBM_PEAK_GBS,
                   "penalty": ("fused into the top-K kernel" if WORKLOADS[a.workload]["cfg"].get("RepeatPenalty", 1.0) != 1.0
                               and WORKLOADS[a.workload]["cfg"].get("TopK", 0) > 0 else "none"),
                   "rows_fast_path": r["fast_frac"], "rows_replay_path": r["replay_frac"]},
        "roofline": {"bound": "hbm", "kernel": DOMINANT_KERNEL[a.workload],
                     "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": read_traffic(a.workload),
                     "kernel_us": 1e3 * r["kernel_ms"], "bytes_per_launch": r["step_bytes"]},
    }
    if "parity" in r:
        out["parity"] = r["parity"]
    if not a.no_north_star:
        # other top-K settings of the same shape: a larger K, and Top-P = 1 (slot-order draw)
        extra = {}
        for name in EXTRA:
            if name == a.workload:
                continue
            o = run_gpu(name, MIN_TIMED, min(a.warmup, 20), a.eager, check=not a.no_check)
            ob = o["step_bytes"] / (o["kernel_ms"] * 1e-3) / 1e9
            extra[name] = {"workload": WORKLOADS[name]["desc"], "steps": o["steps"],
                           "rows_per_s": o["rows"] * o["steps"] / o["elapsed"],
                           "us_per_step": 1e6 * o["elapsed"] / o["steps"], "kernel_us": 1e3 * o["kernel_ms"],
                           "hbm_frac": ob / HBM_PEAK_GBS, "rows_fast_path": o["fast_frac"],
                           "rows_exact_path": o["replay_frac"], "parity": o.get("parity")}
        out["extra_workloads"] = extra
    if NORTH_STAR != a.workload and not a.no_north_star:
        # the target shape: B=256 x V=262144 fp32, top-k 64 / top-p 0.95
        n = run_gpu(NORTH_STAR, steps, min(a.warmup, 20), a.eager, check=not a.no_check)
        nb = n["step_bytes"] / (n["kernel_ms"] * 1e-3) / 1e9
        out["north_star"] = {"workload": WORKLOADS[NORTH_STAR]["desc"], "steps": n["steps"],
                             "rows_per_s": n["rows"] * n["steps"] / n["elapsed"],
                             "us_per_step": 1e6 * n["elapsed"] / n["steps"],
                             "kernel_us": 1e3 * n["kernel_ms"], "achieved_GBs": nb,
                             "hbm_frac": nb / HBM_PEAK_GBS, "target_frac": 0.60,
                             "rows_fast_path": n["fast_frac"], "parity": n.get("parity")}
    if a.others:
        others = {}
        for name in WORKLOADS:
            if name == a.workload:
                continue
            o = run_gpu(name, max(200, a.steps // 4), 20, a.eager)
            others[name] = {"rows_per_s": o["rows"] * o["steps"] / o["elapsed"],
                            "us_per_step": 1e6 * o["elapsed"] / o["steps"],
                            "kernel_us": 1e3 * o["kernel_ms"],
                            "kernel_hbm_frac": o["step_bytes"] / (o["kernel_ms"] * 1e-3) / 1e9
                            / HBM_PEAK_GBS}
        for B in (1, 16):
            others[f"lmhead_b{B}"] = run_lmhead(B, 200, 10)
        others["lmhead_b1_gguf_layout"] = run_lmhead(1, 200, 10, packed=False)
        others["host_process_b1"] = run_host_process()
        others["host_process_b1_penalised"] = run_host_process(penalised=True)
        for fmt in ("q8_0", "f16"):
            others[f"lmhead_{fmt}_norm_b1"] = run_lmhead(1, 200, 10, fmt=fmt, norm=True)
        out["other_workloads"] = others
    if a.copy_calibration:
        copy_calibration()
    if not a.no_cpu:
        L, hist = make_inputs(a.workload)
        out["cpu_baseline"] = cpu_baseline(a.workload, L, hist, a.cpu_seconds)
        nt = host_threads()
        if nt > 1:
            out["cpu_baseline_all_cores"] = cpu_baseline(a.workload, L, hist, a.cpu_seconds / 2, threads=nt)
        out["reference_readback"] = readback_cost(r["rows"], r["vocab"])
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
