#!/usr/bin/env python
"""Benchmark of PackBalance's training hot path on one MI355X.

Headline (``value``): useful tokens/s of the 100M Llama packed-2048 training
step (4 packs of 2048 tokens per step, heavy-tail lognormal documents packed
best-fit-decreasing, bf16 autocast with fp32 master weights, clip + fused
AdamW) -- the semantics of the reference's ``profiling/bench_train.py:54-163``:
useful tok/s = sum of pack tokens / sum of timed step seconds.  The corpus is a
synthetic uint32 token store resident in HBM; each step's packs are built on
the device from it (``pb_pack_tensors``) as the step's first work, the part
of the reference's timed step that loads and copies its micro-batches.

Kernel figures (HIP events around each C-ABI launch, on the stream the kernel
runs on):
  attention  cfg3 masked GQA attention fwd+bwd, 12*D*Hq*P FLOPs (P = allowed pairs)
  lmhead_ce  cfg4 fused LM-head CE fwd+bwd, 6*N*V*D FLOPs, vocab chunk 8192 (the
             configuration's), no full logits; vocab chunk 32768 and a forward that
             keeps the bf16 logits (outside cfg4's rule) reported as labelled variants
  ce_rows    one cfg4 vocab chunk [16384 x 8192] bf16 through the row CE kernel
  rmsnorm / swiglu   cfg5 fwd and bwd, algorithmic bytes moved
The ``roofline`` object is document-masked attention fwd+bwd at cfg3 (MFMA-bound),
the headline "masked-attn TFLOP/s": ``achieved`` = 12*D*Hq*P FLOPs per
forward+backward / the summed HIP-event durations of the two entry points
(pb_attn_fwd: the forward kernel; pb_attn_bwd: at cfg3 the delta, dK/dV
(storing dS) and dQ-from-dS kernels);
``traffic`` = HBM-side bytes of the same kernels per fwd+bwd from the committed
rocprofv3 FETCH_SIZE / WRITE_SIZE summary (profiles/attention_cfg3_hbm_counters.txt).

``cpu_baseline`` times the reference's eager fp32 CPU path, restated in the
test oracle, on this host's cores: the cfg2 step over its 4 packs (the
headline), and in ``cpu_baseline.kernels`` eager attention on one cfg3 pack
(scaled by allowed pairs), chunked CE on one cfg4 vocab chunk (scaled by V)
and RMSNorm / SwiGLU at cfg5 full size.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--skip-cpu] [--skip-kernels]
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBPS = 8000.0  # MI355X HBM3E


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model_name() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


# Kernels of the cfg3 attention entry points (namespace of every attention kernel).
ATTN_KERNELS = "pb::attn::"


def counter_traffic(kernel_substr: str, summary: str = "attention_cfg3_hbm_counters.txt"):
    """HBM-side bytes per call of the kernels whose name contains ``kernel_substr``
    (summed over them), from a committed rocprofv3 counter summary.

    The summary lists calibrated bytes per dispatch (the calibration factor is
    written at its top); None when it is absent or names no such kernel.
    """
    path = ROOT / "profiles" / summary
    total, found = 0.0, False
    try:
        for line in path.read_text().splitlines():
            if line.startswith("#") or kernel_substr not in line:
                continue
            total += float(line.split()[2]) * 1e9
            found = True
    except (OSError, ValueError, IndexError):
        return None
    return total if found else None


# ---------------------------------------------------------------- timing
def events_ms(launch, iters: int, flush=None) -> float:
    """Mean duration (ms) of `launch()` over `iters` calls, each bracketed by events."""
    import torch

    total = 0.0
    for _ in range(iters):
        if flush is not None:
            flush()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        launch()
        e.record()
        e.synchronize()
        total += s.elapsed_time(e)
    return total / iters


def make_flush(dev):
    import torch

    buf = torch.empty(512 * 1024 * 1024 // 4, dtype=torch.float32, device=dev)

    def flush():
        buf.fill_(1.0)  # evicts the 256 MB last-level cache between HBM-bound launches

    return flush


# ---------------------------------------------------------------- cfg2 train step
def train_step_bench(steps: int, warmup: int, dev, use_graph: bool = True, streams: int = 2,
                     packs_per_micro_batch: int = 2):
    import numpy as np
    import torch

    from packbalance_amd.data import workloads as W
    from packbalance_amd.model.llama import cfg2_model, count_parameters
    from packbalance_amd.model.step import TrainStep

    from packbalance_amd.data.device_packs import DeviceTokenStore, build_pack_batch

    cfg = cfg2_model()
    plan = W.cfg2_steps(warmup + steps)
    # Synthetic corpus: every document of the run, uniform token ids, in one
    # uint32 token store resident in HBM; each step's packs are (start, length)
    # segments of it and are built on the device inside the step.
    rng = np.random.default_rng(0)
    n_tok = sum(n for st in plan for p in st for n in p)
    store = DeviceTokenStore(rng.integers(0, cfg.vocab_size, size=n_tok).astype(np.uint32), dev)
    step_packs, pos = [], 0
    for st in plan:
        packs = []
        for p in st:
            packs.append([(pos + sum(p[:i]), n) for i, n in enumerate(p)])
            pos += sum(p)
        step_packs.append(packs)
    # The step's 4 packs run as micro-batches of `packs_per_micro_batch` packs
    # ([k, 2048] each; the step's gradient is the same sum over packs), and the
    # micro-batches run concurrently on `streams` streams (one fp32 gradient
    # slot each, summed by the optimizer's norm pass).
    ts = TrainStep(cfg, dev, store=store, streams=streams,
                   packs_per_micro_batch=packs_per_micro_batch)
    model = ts.model
    if use_graph:
        ts.capture_packs(step_packs[0])
        run = lambda i: ts.replay_packs(step_packs[i])  # noqa: E731
    else:
        run = lambda i: ts.eager_packs(step_packs[i])  # noqa: E731
    for i in range(warmup):
        run(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(warmup, warmup + steps):
        run(i)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    useful = sum(n for st in plan[warmup:] for p in st for n in p)
    flops = sum(W.step_flops(cfg, st) for st in plan[warmup:])
    res = {
        "tok_s": useful / dt,
        "ms_per_step": dt / steps * 1e3,
        "useful_tokens": useful,
        "params": count_parameters(model),
        "model_tflops": flops / dt / 1e12,
        "hip_graph": use_graph,
        "packs_built_on_device": True,
        "micro_batch_streams": len(ts.streams) or 1,
        "packs_per_micro_batch": ts.k,
        "lm_head_logits_kept": ts.keep_logits_bytes >= cfg.vocab_size * ts.k * 2048 * 2,
    }
    # The first timed step's 4 packs, on the host, for the CPU baseline.
    first = build_pack_batch(store, step_packs[warmup], 2048)
    cpu_step = W.PackBatch(first["input_ids"].cpu(), first["labels"].cpu(),
                           first["position_ids"].cpu(), first["doc_ids"].cpu(), plan[warmup])
    return res, model, cfg, cpu_step


# ---------------------------------------------------------------- cpu baseline
def _host_desc() -> str:
    import torch

    return (f"cpu {cpu_model_name()}, affinity {len(os.sched_getaffinity(0))} cores, "
            f"{torch.get_num_threads()} torch threads")


def cpu_baseline(model, cfg, batch) -> dict:
    """The reference's eager fp32 CPU path restated (oracle/model.py) on this host's
    cores: one cfg2 step -- fwd+bwd of each of its 4 packs, then clip + AdamW."""
    import torch

    from oracle import model as OM

    params = OM.cpu_params(model)
    b = batch.to("cpu")
    t0 = time.perf_counter()
    for p in range(b.input_ids.shape[0]):
        sl = slice(p, p + 1)
        loss = OM.loss(params, cfg, b.input_ids[sl], b.labels[sl], b.position_ids[sl],
                       b.doc_ids[sl])
        (loss / b.useful_tokens).backward()
    t_fb = time.perf_counter() - t0
    opt = torch.optim.AdamW(list(params.values()), lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1)
    t0 = time.perf_counter()
    torch.nn.utils.clip_grad_norm_(list(params.values()), 1.0)
    opt.step()
    t_opt = time.perf_counter() - t0
    step_s = t_fb + t_opt
    return {
        "value": b.useful_tokens / step_s,
        "unit": "tok/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"one whole cfg2 step (the first timed step's 4 packs, {b.useful_tokens} "
                   f"tokens): fwd+bwd {t_fb:.2f} s + clip/AdamW {t_opt:.2f} s of the eager fp32 "
                   "CPU path on the 100M model; " + _host_desc()),
    }


def cpu_kernel_baselines() -> dict:
    """Per-kernel CPU baselines of the reference's eager fp32 functions (restated in
    the oracle): eager_attention, chunked_linear_cross_entropy, rmsnorm_reference and
    swiglu_reference, fwd+bwd by autograd: cfg5 at full size, cfg3 and cfg4 on one
    pack / one vocab chunk (a few seconds each on the GPU box's host) scaled
    linearly to the whole config."""
    import torch
    import torch.nn.functional as F

    from oracle import model as OM
    from packbalance_amd.data import workloads as W

    out = {}
    g = torch.Generator().manual_seed(0)
    # cfg3: pack 1 (all heads), scaled to the 8 packs by allowed pairs.
    packs = W.cfg3_packs()
    S, Hq, Hkv, D = 8192, 32, 8, 128
    hq = Hq
    doc = W.doc_ids_from_lengths(packs[1:2], S)
    q = torch.randn(1, Hq, S, D, generator=g).requires_grad_(True)
    k = torch.randn(1, Hkv, S, D, generator=g).requires_grad_(True)
    v = torch.randn(1, Hkv, S, D, generator=g).requires_grad_(True)
    t0 = time.perf_counter()
    o = OM._eager_attention(q, k, v, doc)
    o.backward(torch.ones_like(o))
    dt = time.perf_counter() - t0
    p1, pall = W.attention_pairs(packs[1:2]), W.attention_pairs(packs)
    scale = pall / p1
    out["attention"] = {"tflops": 12.0 * D * hq * p1 / dt / 1e12, "unit": "TFLOP/s",
                        "cfg3_fwd_bwd_s": dt * scale,
                        "sample": f"eager_attention fwd+bwd on cfg3 pack 1 ({len(packs[1])} "
                                  f"documents, {p1} pairs per head, 32 query heads) in {dt:.2f} s; "
                                  f"x{scale:.2f} by allowed pairs to the 8 packs"}
    del q, k, v, o
    # cfg4: chunked CE (token chunks of 1024) of all 16384 tokens against one 8192-row
    # vocab chunk, scaled by V.
    N, V, Dm, n, vc = 16384, 128256, 4096, 16384, 8192
    x = torch.randn(n, Dm, generator=g).requires_grad_(True)
    w = (torch.randn(vc, Dm, generator=g) * 0.02).requires_grad_(True)
    t = torch.randint(0, vc, (n,), generator=g)
    t0 = time.perf_counter()
    OM._chunked_ce(x, w, t, 1024, 0.0).backward()
    dt = time.perf_counter() - t0
    scale = (N / n) * (V / vc)
    out["lmhead_ce"] = {"tflops": 6.0 * n * vc * Dm / dt / 1e12, "unit": "TFLOP/s",
                        "cfg4_fwd_bwd_s": dt * scale,
                        "sample": f"chunked_linear_cross_entropy fwd+bwd, x [16384, 4096] against "
                                  f"one 8192-row vocab chunk in {dt:.2f} s; x{scale:.2f} to cfg4"}
    del x, w
    # cfg5 at full size (fp32, the reference's CPU dtype).
    R, H, r = 32768, 4096, 32768
    x = torch.randn(r, H, generator=g).requires_grad_(True)
    wn = (torch.randn(H, generator=g) * 0.1 + 1.0).requires_grad_(True)
    t0 = time.perf_counter()
    y = OM._rmsnorm(x, wn, 1e-5)
    y.backward(torch.ones_like(y))
    dt = time.perf_counter() - t0
    nbytes = (2 * r * H * 2 + H * 2 + r * 4) + (3 * r * H * 2 + r * 4 + 2 * H * 2)
    out["rmsnorm"] = {"gbps": nbytes / dt / 1e9, "unit": "GB/s (cfg5's bf16 algorithmic bytes)",
                      "cfg5_fwd_bwd_s": dt * R / r,
                      "sample": f"rmsnorm_reference fwd+bwd (autograd, fp32) at cfg5 full size "
                                f"in {dt:.2f} s"}
    del x, y
    R, Fd, r = 32768, 14336, 32768
    gt = torch.randn(r, Fd, generator=g).requires_grad_(True)
    up = torch.randn(r, Fd, generator=g).requires_grad_(True)
    t0 = time.perf_counter()
    y = F.silu(gt) * up
    y.backward(torch.ones_like(y))
    dt = time.perf_counter() - t0
    out["swiglu"] = {"gbps": 8 * r * Fd * 2 / dt / 1e9, "unit": "GB/s (cfg5's bf16 algorithmic bytes)",
                     "cfg5_fwd_bwd_s": dt * R / r,
                     "sample": f"swiglu_reference fwd+bwd (autograd, fp32) at cfg5 full size "
                               f"in {dt:.2f} s"}
    out["host"] = _host_desc()
    return out


# ---------------------------------------------------------------- kernels
def _attention_timing(dev, iters: int, packs, B: int, S: int, Hq: int, Hkv: int, D: int):
    """Event-timed pb_attn_fwd / pb_attn_bwd (bf16, plans built beforehand) on `packs`:
    (fwd_ms, bwd_ms, fwd FLOPs, bwd FLOPs, allowed pairs per head, doc ids)."""
    import torch

    from packbalance_amd import _native as N
    from packbalance_amd.data import workloads as W
    from packbalance_amd.model import attention as A

    doc = W.doc_ids_from_lengths(packs, S).to(dev)
    torch.manual_seed(0)
    q = torch.randn(B, S, Hq, D, device=dev, dtype=torch.bfloat16).transpose(1, 2)
    k = torch.randn(B, S, Hkv, D, device=dev, dtype=torch.bfloat16).transpose(1, 2)
    v = torch.randn(B, S, Hkv, D, device=dev, dtype=torch.bfloat16).transpose(1, 2)
    do = torch.randn(B, S, Hq, D, device=dev, dtype=torch.bfloat16).transpose(1, 2)
    plans = A._plans(doc, Hq, Hkv, D, None)
    out = torch.empty(B, S, Hq, D, device=dev, dtype=torch.bfloat16).transpose(1, 2)
    lse = torch.empty(B, Hq, S, device=dev, dtype=torch.float32)
    dq = torch.empty_like(out)
    dk = torch.empty(B, S, Hkv, D, device=dev, dtype=torch.bfloat16).transpose(1, 2)
    dv = torch.empty_like(dk)
    ws = torch.empty(plans["workspace"], dtype=torch.uint8, device=dev)
    fws = torch.empty(max(1, plans["fwd_workspace"]), dtype=torch.uint8, device=dev)
    sc = 1.0 / D ** 0.5
    st = N.stream_ptr(q)
    pf, pq, pk = plans[A.FWD], plans[A.BWD_Q], plans[A.BWD_KV]

    def fwd():
        N.call("pb_attn_fwd", N.BHSD.of(q), N.BHSD.of(k), N.BHSD.of(v), N.BHSD.of(out),
               lse.data_ptr(), fws.data_ptr(), doc.data_ptr(), doc.stride(0),
               pf.counts.data_ptr(), pf.lists.data_ptr(), B, Hq, Hkv, S, D, sc, N.PB_BF16, st)

    def bwd():
        N.call("pb_attn_bwd", N.BHSD.of(q), N.BHSD.of(k), N.BHSD.of(v), N.BHSD.of(out),
               N.BHSD.of(do), N.BHSD.of(dq), N.BHSD.of(dk), N.BHSD.of(dv), lse.data_ptr(),
               ws.data_ptr(), doc.data_ptr(), doc.stride(0), pq.counts.data_ptr(),
               pq.lists.data_ptr(), pk.counts.data_ptr(), pk.lists.data_ptr(), B, Hq, Hkv, S, D,
               sc, N.PB_BF16, st)

    fwd()
    bwd()
    torch.cuda.synchronize()
    t_f = events_ms(fwd, iters)
    t_b = events_ms(bwd, iters)
    pairs = float(W.attention_pairs(packs))
    return t_f, t_b, 4.0 * D * Hq * pairs, 8.0 * D * Hq * pairs, pairs, doc


def attention_kernels(dev, iters: int) -> dict:
    from packbalance_amd.data import workloads as W
    from packbalance_amd.model import attention as A

    packs = W.cfg3_packs()
    B, S, Hq, Hkv, D = 8, 8192, 32, 8, 128
    t_f, t_b, f_fwd, f_bwd, pairs, doc = _attention_timing(dev, iters, packs, B, S, Hq, Hkv, D)
    # Secondary, tile-size dependent: every 128 x 128 block with at least one
    # allowed pair (FlexAttention's PARTIAL + FULL blocks) counted as dense.
    blocks = 0
    for b in range(B):
        t = A.doc_block_tables(doc[b:b + 1], 1, 128)
        blocks += int(t["kv_num_blocks"].sum()) + int(t["full_kv_num_blocks"].sum())
    f_blk = 12.0 * D * Hq * 128 * 128 * blocks
    return {
        "workload": "cfg3: 8 packs x 8192, Hq 32, Hkv 8, D 128, bf16, pack 0 dense",
        "allowed_pairs_per_head": pairs,
        "fwd_ms": t_f, "bwd_ms": t_b,
        "fwd_tflops": f_fwd / t_f / 1e9, "bwd_tflops": f_bwd / t_b / 1e9,
        "fwd_bwd_tflops": (f_fwd + f_bwd) / (t_f + t_b) / 1e9,
        "frac_bf16_peak": (f_fwd + f_bwd) / (t_f + t_b) / 1e9 / PEAK_BF16_TFLOPS,
        "fwd_frac_bf16_peak": f_fwd / t_f / 1e9 / PEAK_BF16_TFLOPS,
        "flops_per_fwd_bwd": f_fwd + f_bwd,
        "nonempty_blocks_128": blocks,
        "effective_block_tflops": f_blk / (t_f + t_b) / 1e9,
        "effective_block_note": "secondary: 12*D*Hq*128^2 per non-empty 128x128 block "
                                "(PARTIAL+FULL) over fwd+bwd time; tile-size dependent",
    }


def attention_cfg2_kernels(dev, iters: int) -> dict:
    """The attention of one cfg2 micro-batch (the first step's first two packs as one
    [2, 2048] batch, Hq 12, Hkv 4, D 64, bf16), as each layer of the training step runs
    it.  Labelled, not the roofline: a small, launch- and VALU-bound problem."""
    from packbalance_amd.data import workloads as W

    packs = W.cfg2_steps(1)[0][:2]
    B, S, Hq, Hkv, D = 2, 2048, 12, 4, 64
    t_f, t_b, f_fwd, f_bwd, pairs, _ = _attention_timing(dev, iters, packs, B, S, Hq, Hkv, D)
    return {
        "workload": "cfg2 micro-batch: [2, 2048] (step 1, packs 0-1), Hq 12, Hkv 4, D 64, bf16",
        "allowed_pairs_per_head": pairs,
        "fwd_us": t_f * 1e3, "bwd_us": t_b * 1e3,
        "fwd_bwd_tflops": (f_fwd + f_bwd) / (t_f + t_b) / 1e9,
        "frac_bf16_peak": (f_fwd + f_bwd) / (t_f + t_b) / 1e9 / PEAK_BF16_TFLOPS,
    }


PEAK_FP32_TFLOPS = 157.3  # MI355X dense fp32


def attention_f32_kernels(dev, iters: int) -> dict:
    """The fp32 attention path (fp32 q/k/v without autocast, where the reference's
    FlexAttention computes in fp32) at the cfg2 attention shape: the first step's
    first [2, 2048] micro-batch, Hq 12, Hkv 4, D 64.  Labelled, not a headline: these
    kernels are the precision path (fp32 operands on v_mfma_f32_32x32x2_f32)."""
    import torch

    from packbalance_amd import _native as N
    from packbalance_amd.data import workloads as W

    packs = W.cfg2_steps(1)[0][:2]
    B, S, Hq, Hkv, D = 2, 2048, 12, 4, 64
    doc = W.doc_ids_from_lengths(packs, S).to(dev)
    g = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(B, S, Hq, D, device=dev, generator=g).transpose(1, 2)
    k = torch.randn(B, S, Hkv, D, device=dev, generator=g).transpose(1, 2)
    v = torch.randn(B, S, Hkv, D, device=dev, generator=g).transpose(1, 2)
    do = torch.randn(B, S, Hq, D, device=dev, generator=g).transpose(1, 2)
    out = torch.empty(B, S, Hq, D, device=dev).transpose(1, 2)
    dq = torch.empty_like(out)
    dk = torch.empty(B, S, Hkv, D, device=dev).transpose(1, 2)
    dv = torch.empty_like(dk)
    lse = torch.empty(B, Hq, S, device=dev)
    bws = torch.empty(N.lib().pb_attn_bwd_f32_workspace_bytes(B, Hq, Hkv, S, D),
                      dtype=torch.uint8, device=dev)
    sc, st = 1.0 / D ** 0.5, N.stream_ptr(q)

    def fwd():
        N.call("pb_attn_fwd_f32", N.BHSD.of(q), N.BHSD.of(k), N.BHSD.of(v), N.BHSD.of(out),
               lse.data_ptr(), doc.data_ptr(), doc.stride(0), B, Hq, Hkv, S, D, sc, st)

    def bwd():
        N.call("pb_attn_bwd_f32", N.BHSD.of(q), N.BHSD.of(k), N.BHSD.of(v), N.BHSD.of(out),
               N.BHSD.of(do), N.BHSD.of(dq), N.BHSD.of(dk), N.BHSD.of(dv), lse.data_ptr(),
               bws.data_ptr(), doc.data_ptr(), doc.stride(0), B, Hq, Hkv, S, D, sc, st)

    fwd()
    bwd()
    torch.cuda.synchronize()
    t_f = events_ms(fwd, iters)
    t_b = events_ms(bwd, iters)
    pairs = float(W.attention_pairs(packs))
    f_fwd, f_bwd = 4.0 * D * Hq * pairs, 8.0 * D * Hq * pairs
    return {
        "workload": "cfg2 attention shape in fp32: [2, 2048] micro-batch, Hq 12, Hkv 4, D 64",
        "allowed_pairs_per_head": pairs,
        "fwd_ms": t_f, "bwd_ms": t_b,
        "fwd_bwd_tflops": (f_fwd + f_bwd) / (t_f + t_b) / 1e9,
        "frac_fp32_peak": (f_fwd + f_bwd) / (t_f + t_b) / 1e9 / PEAK_FP32_TFLOPS,
        "note": "precision path (pb_attn_fwd_f32 / pb_attn_bwd_f32): fp32 operands on the fp32 "
                "matrix cores; fraction of the 157.3 TFLOP/s dense fp32 peak",
    }


def lmhead_ce_kernels(dev, iters: int, vchunk: int = 8192, stored: bool = False) -> dict:
    import torch

    from packbalance_amd.kernels.fused_ce import (linear_cross_entropy, logits_budget,
                                                  stores_logits, vocab_chunk, vocab_chunk_rows)

    Nt, V, D = 16384, 128256, 4096
    torch.manual_seed(0)
    x = torch.randn(Nt, D, device=dev, dtype=torch.bfloat16).requires_grad_(True)
    w = (torch.randn(V, D, device=dev) * 0.02).to(torch.bfloat16).requires_grad_(True)
    t = torch.randint(0, V, (Nt,), device=dev)
    t[torch.rand(Nt, device=dev) < 0.01] = -100
    holder = {}

    def fwd():
        holder["loss"] = linear_cross_entropy(x, w, t)

    def bwd():
        holder["loss"].backward()

    with vocab_chunk_rows(vchunk), logits_budget((16 << 30) if stored else 0):
        fwd()
        bwd()
        torch.cuda.synchronize()
        tf = tb = 0.0
        for _ in range(iters):
            x.grad = None
            w.grad = None
            tf += events_ms(fwd, 1)
            tb += events_ms(bwd, 1)
        chunk = vocab_chunk(Nt, V)
        kept = stores_logits(Nt, V)
    tf /= iters
    tb /= iters
    flops = 6.0 * Nt * V * D
    return {
        "workload": "cfg4: x [16384, 4096] bf16, W [128256, 4096] bf16, 1% ignored",
        "vocab_chunk": chunk,
        "logits_stored": kept,
        "fwd_ms": tf, "bwd_ms": tb,
        "tflops": flops / (tf + tb) / 1e9,
        "frac_bf16_peak": flops / (tf + tb) / 1e9 / PEAK_BF16_TFLOPS,
        "note": ("variant outside cfg4's no-full-logits rule: the forward keeps the bf16 "
                 "logits (4.2 GB) and the backward forms dlogits from them in a memory-bound "
                 "pass; 6NVD executed and counted" if kept else
                 "no full logits (cfg4's rule): fwd 2NVD + bwd 6NVD executed (logits "
                 "recomputed once); 6NVD counted"),
        "kernels": ("lse and dlogits on this build's MFMA kernels (pb_lmhead_ce_fwd, "
                    "pb_lmhead_ce_dlogits); dx and dW as plain hipBLASLt GEMMs (torch)"),
    }


def lmhead_ce_f32_kernels(dev, iters: int) -> dict:
    """The fp32 LM-head CE path (fp32 x and W outside bf16 autocast, where the reference
    computes fp32 logits): cfg4's shape with fp32 operands.  Labelled, not a headline:
    fp32 library GEMMs (torch -> hipBLASLt) over token-row chunks of fp32 logits
    (<= 1 GiB each) with the row CE kernel; fraction of the fp32 peak."""
    import torch

    from packbalance_amd.kernels.fused_ce import linear_cross_entropy

    Nt, V, D = 16384, 128256, 4096
    torch.manual_seed(0)
    x = torch.randn(Nt, D, device=dev).requires_grad_(True)
    w = (torch.randn(V, D, device=dev) * 0.02).requires_grad_(True)
    t = torch.randint(0, V, (Nt,), device=dev)
    t[torch.rand(Nt, device=dev) < 0.01] = -100
    holder = {}

    def fwd():
        holder["loss"] = linear_cross_entropy(x, w, t)

    def bwd():
        holder["loss"].backward()

    fwd()
    bwd()
    torch.cuda.synchronize()
    tf = tb = 0.0
    for _ in range(iters):
        x.grad = None
        w.grad = None
        tf += events_ms(fwd, 1)
        tb += events_ms(bwd, 1)
    tf /= iters
    tb /= iters
    flops = 6.0 * Nt * V * D
    return {
        "workload": "cfg4 shape in fp32: x [16384, 4096], W [128256, 4096] fp32, 1% ignored",
        "fwd_ms": tf, "bwd_ms": tb,
        "tflops": flops / (tf + tb) / 1e9,
        "frac_fp32_peak": flops / (tf + tb) / 1e9 / PEAK_FP32_TFLOPS,
        "note": "precision path: fp32 logits GEMM per token-row chunk, row CE kernel, fp32 "
                "dx / dW GEMMs (6NVD counted); fraction of the 157.3 TFLOP/s dense fp32 peak",
    }


def ce_rows_kernel(dev, iters: int, flush) -> dict:
    import torch

    from packbalance_amd import _native as N

    m, v = 16384, 8192
    torch.manual_seed(0)
    logits = torch.randn(m, v, device=dev).to(torch.bfloat16)
    t = torch.randint(0, v, (m,), device=dev)
    loss = torch.empty(m, device=dev)
    lse = torch.empty(m, device=dev)
    dl = torch.empty_like(logits)
    st = N.stream_ptr(logits)

    def launch():
        N.call("pb_ce_rows", logits.data_ptr(), v, 1, N.PB_BF16, t.data_ptr(), loss.data_ptr(),
               lse.data_ptr(), dl.data_ptr(), m, v, -100, 0.0, st)

    launch()
    ms = events_ms(launch, iters, flush)
    nbytes = 2 * m * v * 2 + m * 8 + 2 * m * 4
    return {"workload": "one cfg4 vocab chunk: logits [16384, 8192] bf16 -> loss, lse, dlogits",
            "ms": ms, "bytes": nbytes, "gbps": nbytes / ms / 1e6,
            "frac_hbm_peak": nbytes / ms / 1e6 / PEAK_HBM_GBPS}


def norm_act_kernels(dev, iters: int, flush) -> dict:
    import torch

    from packbalance_amd import _native as N

    out = {}
    R, H = 32768, 4096
    torch.manual_seed(0)
    x = torch.randn(R, H, device=dev, dtype=torch.bfloat16)
    w = (torch.randn(H, device=dev) * 0.1 + 1.0).to(torch.bfloat16)
    dy = torch.randn(R, H, device=dev, dtype=torch.bfloat16)
    y = torch.empty_like(x)
    dx = torch.empty_like(x)
    dw = torch.empty_like(w)
    rstd = torch.empty(R, device=dev)
    ws = torch.empty(N.lib().pb_rmsnorm_bwd_workspace_bytes(R, H) // 4, device=dev)
    st = N.stream_ptr(x)

    def rf():
        N.call("pb_rmsnorm_fwd", x.data_ptr(), H, N.PB_BF16, w.data_ptr(), N.PB_BF16, y.data_ptr(),
               H, rstd.data_ptr(), R, H, 1e-5, st)

    def rb():
        N.call("pb_rmsnorm_bwd", dy.data_ptr(), H, x.data_ptr(), H, N.PB_BF16, w.data_ptr(),
               N.PB_BF16, rstd.data_ptr(), dx.data_ptr(), H, dw.data_ptr(), ws.data_ptr(), R, H, st)

    rf()
    rb()
    t_rf = events_ms(rf, iters, flush)
    t_rb = events_ms(rb, iters, flush)
    b_rf = 2 * R * H * 2 + H * 2 + R * 4
    b_rb = 3 * R * H * 2 + R * 4 + 2 * H * 2
    out["rmsnorm"] = {"workload": "cfg5: [32768, 4096] bf16, w bf16", "fwd_ms": t_rf,
                      "bwd_ms": t_rb, "fwd_gbps": b_rf / t_rf / 1e6, "bwd_gbps": b_rb / t_rb / 1e6,
                      "fwd_bwd_gbps": (b_rf + b_rb) / (t_rf + t_rb) / 1e6,
                      "frac_hbm_peak": (b_rf + b_rb) / (t_rf + t_rb) / 1e6 / PEAK_HBM_GBPS}
    del x, dy, y, dx
    R, F = 32768, 14336
    n = R * F
    g = torch.randn(R, F, device=dev, dtype=torch.bfloat16)
    u = torch.randn(R, F, device=dev, dtype=torch.bfloat16)
    d = torch.randn(R, F, device=dev, dtype=torch.bfloat16)
    o = torch.empty_like(g)
    dg = torch.empty_like(g)
    du = torch.empty_like(g)

    def sf():
        N.call("pb_swiglu_fwd", g.data_ptr(), u.data_ptr(), o.data_ptr(), n, N.PB_BF16, st)

    def sb():
        N.call("pb_swiglu_bwd", g.data_ptr(), u.data_ptr(), d.data_ptr(), dg.data_ptr(),
               du.data_ptr(), n, N.PB_BF16, st)

    sf()
    sb()
    t_sf = events_ms(sf, iters, flush)
    t_sb = events_ms(sb, iters, flush)
    out["swiglu"] = {"workload": "cfg5: gate/up [32768, 14336] bf16", "fwd_ms": t_sf,
                     "bwd_ms": t_sb, "fwd_gbps": 3 * n * 2 / t_sf / 1e6,
                     "bwd_gbps": 5 * n * 2 / t_sb / 1e6,
                     "fwd_bwd_gbps": 8 * n * 2 / (t_sf + t_sb) / 1e6,
                     "frac_hbm_peak": 8 * n * 2 / (t_sf + t_sb) / 1e6 / PEAK_HBM_GBPS}
    return out


def copy_calibration(dev, iters: int) -> dict:
    """A plain device copy of known size: the scale reference for HBM byte counters."""
    import torch

    n = 1 << 29  # 1 GiB of bf16
    src = torch.randn(n // 2, device=dev).to(torch.bfloat16).repeat(2)
    dst = torch.empty_like(src)
    ms = events_ms(lambda: dst.copy_(src), iters)
    nbytes = src.numel() * src.element_size()
    return {"bytes_read": nbytes, "bytes_written": nbytes, "ms": ms,
            "gbps": 2 * nbytes / ms / 1e6}


def on_box_peaks(dev, iters: int) -> dict:
    """Practical ceilings measured on this card, reported beside the spec peaks: a large
    bf16 GEMM through torch.mm (hipBLASLt) and a 1 GiB device copy (torch's copy_)."""
    import torch

    n = 8192
    g = torch.Generator(device=dev).manual_seed(0)
    a = torch.randn(n, n, device=dev, dtype=torch.bfloat16, generator=g)
    b = torch.randn(n, n, device=dev, dtype=torch.bfloat16, generator=g)
    c = torch.empty(n, n, device=dev, dtype=torch.bfloat16)
    events_ms(lambda: torch.mm(a, b, out=c), 3)  # library warm-up
    ms = events_ms(lambda: torch.mm(a, b, out=c), iters)
    del a, b, c
    copy = copy_calibration(dev, iters)
    return {"gemm_bf16": {"shape_mnk": [n, n, n], "ms": ms, "tflops": 2 * n ** 3 / ms / 1e9,
                          "library": "torch.mm -> hipBLASLt"},
            "copy": {"bytes": copy["bytes_read"], "ms": copy["ms"], "gbps": copy["gbps"],
                     "library": "torch copy_ (kernels with non-temporal streams can exceed it)"}}


def add_on_box_fractions(kernels: dict, peaks: dict) -> None:
    """frac_on_box: each kernel's headline rate over the matching on-box ceiling."""
    gemm, copy = peaks["gemm_bf16"]["tflops"], peaks["copy"]["gbps"]
    rates = {"attention": ("fwd_bwd_tflops", gemm), "lmhead_ce": ("tflops", gemm),
             "lmhead_ce_chunk32768": ("tflops", gemm),
             "lmhead_ce_stored_logits": ("tflops", gemm), "ce_rows": ("gbps", copy),
             "rmsnorm": ("fwd_bwd_gbps", copy), "swiglu": ("fwd_bwd_gbps", copy)}
    for name, (key, peak) in rates.items():
        if name in kernels and key in kernels[name]:
            kernels[name]["frac_on_box"] = kernels[name][key] / peak


# ---------------------------------------------------------------- main
def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--kernel-iters", type=int, default=10)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--skip-kernels", action="store_true")
    ap.add_argument("--eager", action="store_true",
                    help="run the training step eagerly instead of as one captured HIP graph")
    ap.add_argument("--packs-per-micro-batch", type=int, default=2,
                    help="packs run as one [k, 2048] micro-batch (1, 2 or 4)")
    ap.add_argument("--streams", type=int, default=2,
                    help="streams the step's micro-batches run on concurrently (1: one after another)")
    ap.add_argument("--only", choices=["train", "attention", "attention_cfg2", "attention_f32",
                                       "lmhead_ce", "lmhead_ce_f32",
                                       "lmhead_ce_stored",
                                       "ce_rows", "norm_act", "copy", "peaks"],
                    default=None, help="run one part only (for profiling)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(see the sharding design); run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    from packbalance_amd import _native as N

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    N.lib()
    dev = torch.device("cuda:0")
    torch.backends.cuda.matmul.allow_tf32 = True

    if args.only and args.only != "train":
        flush = make_flush(dev)
        fn = {"attention": lambda: attention_kernels(dev, args.kernel_iters),
              "attention_cfg2": lambda: attention_cfg2_kernels(dev, max(20, args.kernel_iters)),
              "attention_f32": lambda: attention_f32_kernels(dev, args.kernel_iters),
              "lmhead_ce": lambda: lmhead_ce_kernels(dev, args.kernel_iters),
              "lmhead_ce_f32": lambda: lmhead_ce_f32_kernels(dev, 2),
              "lmhead_ce_stored": lambda: lmhead_ce_kernels(dev, args.kernel_iters, stored=True),
              "ce_rows": lambda: ce_rows_kernel(dev, args.kernel_iters, flush),
              "norm_act": lambda: norm_act_kernels(dev, args.kernel_iters, flush),
              "copy": lambda: copy_calibration(dev, args.kernel_iters),
              "peaks": lambda: on_box_peaks(dev, args.kernel_iters)}[args.only]
        print(json.dumps({args.only: fn()}), flush=True)
        return 0

    log(f"train step: {args.warmup} warmup + {args.steps} timed steps")
    train, model, cfg, cpu_step = train_step_bench(args.steps, args.warmup, dev,
                                                   use_graph=not args.eager,
                                                   streams=args.streams,
                                                   packs_per_micro_batch=args.packs_per_micro_batch)
    log(f"train: {train['tok_s']:.0f} tok/s, {train['ms_per_step']:.2f} ms/step")
    if args.only == "train":
        print(json.dumps({"train": train}), flush=True)
        return 0

    kernels = {}
    roofline = None
    peaks = None
    if not args.skip_kernels:
        flush = make_flush(dev)
        log("kernels: attention (cfg3)")
        kernels["attention"] = attention_kernels(dev, args.kernel_iters)
        log("kernels: attention at the cfg2 micro-batch shape (labelled)")
        kernels["attention_cfg2"] = attention_cfg2_kernels(dev, max(20, args.kernel_iters))
        log("kernels: attention, fp32 path (cfg2 shape, labelled)")
        kernels["attention_f32"] = attention_f32_kernels(dev, max(2, args.kernel_iters // 2))
        a = kernels["attention"]
        roofline = {"bound": "mfma",
                    "kernel": "document-masked attention fwd+bwd at cfg3: pb_attn_fwd + pb_attn_bwd "
                              "(attn_fwd_pipe; attn_bwd_delta, attn_bwd_dkdv_pairs<128, true>, "
                              "attn_bwd_dq_ds)",
                    "achieved": a["fwd_bwd_tflops"], "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                    "frac": a["fwd_bwd_tflops"] / PEAK_BF16_TFLOPS,
                    "traffic": counter_traffic(ATTN_KERNELS),
                    "algorithmic": "12*D*Hq*P FLOPs per fwd+bwd, P = sum over documents of "
                                   "L(L+1)/2 = %d pairs per head" % a["allowed_pairs_per_head"],
                    "note": f"forward alone {a['fwd_frac_bf16_peak']:.3f} of peak, backward "
                            f"{a['bwd_tflops'] / PEAK_BF16_TFLOPS:.3f} (kernels.attention)"}
        log("kernels: fused LM-head CE (cfg4, vocab chunk 8192)")
        kernels["lmhead_ce"] = lmhead_ce_kernels(dev, max(2, args.kernel_iters // 3), 8192)
        log("kernels: fused LM-head CE (cfg4, vocab chunk 8192, logits kept: variant)")
        kernels["lmhead_ce_stored_logits"] = lmhead_ce_kernels(
            dev, max(2, args.kernel_iters // 3), 8192, stored=True)
        log("kernels: fused LM-head CE (cfg4, vocab chunk 32768)")
        kernels["lmhead_ce_chunk32768"] = lmhead_ce_kernels(dev, max(2, args.kernel_iters // 3),
                                                            32768)
        kernels["lmhead_ce_chunk32768"]["note"] = ("variant: the default budget rule's chunk; "
                                                   "the configuration states 8192")
        log("kernels: LM-head CE, fp32 path (cfg4 shape, labelled)")
        kernels["lmhead_ce_f32"] = lmhead_ce_f32_kernels(dev, 2)
        log("kernels: row CE chunk")
        kernels["ce_rows"] = ce_rows_kernel(dev, args.kernel_iters, flush)
        log("kernels: RMSNorm / SwiGLU (cfg5)")
        kernels.update(norm_act_kernels(dev, args.kernel_iters, flush))
        log("on-box peaks: 8192^3 bf16 GEMM, 1 GiB copy")
        peaks = on_box_peaks(dev, args.kernel_iters)
        add_on_box_fractions(kernels, peaks)

    base = None
    if not args.skip_cpu:
        log("cpu baseline (eager fp32 CPU path): cfg2 step")
        base = cpu_baseline(model, cfg, cpu_step)
        log("cpu baseline: cfg3 attention, cfg4 CE chunk, cfg5 norm / activation")
        base["kernels"] = cpu_kernel_baselines()

    line = {
        "metric": "useful tok/s fwd+bwd (100M, 2048 packed); masked-attn TFLOP/s; CE GB/s",
        "value": train["tok_s"],
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": train["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (lognormal docs, BFD packs, uniform token ids; random-init weights)",
        "config": {
            "workload": "cfg2: 100M Llama (12L, d768, Hq12/Hkv4, ffn2048, vocab32000, tied), "
                        "4 packs x 2048 per step, bf16 autocast + fp32 master, AdamW",
            "global_batch": 4,
            "seq_len": 2048,
            "parallelism": "single GPU",
            "params": train["params"],
            "model_tflops": train["model_tflops"],
            "hip_graph": train["hip_graph"],
            "micro_batch_streams": train["micro_batch_streams"],
            "packs_per_micro_batch": train["packs_per_micro_batch"],
            "lm_head_logits_kept": train["lm_head_logits_kept"],
        },
        "masked_attn_tflops": kernels.get("attention", {}).get("fwd_bwd_tflops"),
        "ce_gbps": kernels.get("ce_rows", {}).get("gbps"),
        "roofline": roofline,
        "on_box_peaks": peaks,
        "cpu_baseline": base,
        "kernels": kernels,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
