"""Benchmark of the DSA hot path on one MI355X.

Headline (``value``): lightning_indexer (score + stable top-k) rows/s on
BASELINE config 2 -- BSND 1x8192, 64 indexer heads, D=128, top-k 2048, causal.
One step = one lightning_indexer call over the whole 8192-row batch, inputs
resident in HBM. The same JSON line carries:
  roofline      -- the indexer score kernel (dominant) against bf16 dense MFMA peak,
                   timed with HIP events on the launch stream;
  cpu_baseline  -- the numpy oracle (a port of the reference goldens) on this host:
                   C2 (the headline's figure) on a stride sample of rows, plus C1 and C4
                   in full and C3 / C5 on stride samples, each beside its GPU figure;
  breakdown     -- top-k kernel, SFA prefill (config 3), SFA paged decode (config 4),
                   the SFA backward at the reference's grad perf shape, the sparse LI
                   grad KL loss at its target shape, and the TND indexer->SFA pipeline
                   (config 5).

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--quick]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
METRIC = "indexer+topk rows/s & TFLOP/s; SFA fwd TFLOP/s (prefill), KV GB/s (decode), % roof"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def timed(fn, steps, warmup, torch):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def warm(fn, torch, seconds=0.2):
    """Untimed calls for about `seconds` of GPU work, so the timed region sees the
    steady-state clocks the card settles at under this load (the first few calls
    after a pause run ~15% slower)."""
    fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        fn()
        torch.cuda.synchronize()


def event_time(fns, reps, torch):
    """Average device time (ms) of each callable: `reps` back-to-back calls between
    two HIP events on the current stream (the stream every kernel here is launched
    on). Back-to-back calls keep the GPU fed, so the host's per-call enqueue time
    (Python + ctypes, ~10-15 us) does not show up as device time."""
    out = []
    for f in fns:
        f()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            f()
        e1.record()
        torch.cuda.synchronize()
        out.append(e0.elapsed_time(e1) / reps)
    return out


def cpu_host_info():
    """Host cores this process may run on, the CPU model and numpy's BLAS threads."""
    cores = len(os.sched_getaffinity(0))
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    blas = []
    try:
        from threadpoolctl import threadpool_info
        blas = [f"{i.get('internal_api')}:{i.get('num_threads')}" for i in threadpool_info()
                if i.get("user_api") == "blas"]
    except Exception:
        pass
    return cores, model, blas


def cpu_baselines(torch, W, gpu):
    """The numpy oracle (a port of the reference goldens, the same per-row loops) on this
    host, on the same seeded inputs as the GPU figures: C1 and C4 in full, C2, C3 and C5
    on deterministic stride samples of rows spanning the causal triangle (BASELINE.md
    section 3). Each entry gives CPU rows/s beside the GPU rows/s of the same config."""
    import numpy as np
    from oracle import lightning_indexer_ref as LIO
    from oracle import sparse_flash_attention_ref as SFAO
    f = lambda t: t.float().cpu().numpy()
    out = {}

    def entry(name, rows_done, total_rows, dt, stride, gpu_ms, what):
        rps = rows_done / dt
        e = {"cpu_rows_per_s": round(rps, 2), "cpu_s": round(dt, 2), "rows_sampled": rows_done,
             "rows_total": total_rows, "stride": stride, "extrapolated_full_call_s": round(total_rows / rps, 2),
             "sample": what}
        if gpu_ms:
            e["gpu_rows_per_s"] = round(total_rows / (gpu_ms * 1e-3), 1)
        out[name] = e

    # C1: the reference's own CPU shape, every row
    inp = W.indexer_inputs(**W.C1, device="cpu", seed=42)
    q, k, w = f(inp.query), f(inp.key), f(inp.weights)
    t0 = time.perf_counter()
    LIO.li_golden_bsnd(q, k, w, [256], [256], 64, 3, True)
    entry("C1", 256, 256, time.perf_counter() - t0, 1, gpu.get("c1_ms"), "all 256 rows")

    # C2: every 2nd row, from the last (longest) one down, spanning the causal triangle
    c = dict(W.C2)
    inp = W.indexer_inputs(**c, device="cuda:0", seed=42)
    q, k, w = f(inp.query), f(inp.key), f(inp.weights)
    del inp
    S, stride = c["S1"], 2
    rows = [(0, s) for s in range(S - 1, -1, -stride)]
    t0 = time.perf_counter()
    LIO.li_golden_bsnd(q, k, w, [S], [S], c["sparse_count"], 3, True, rows=rows)
    entry("C2", len(rows), S, time.perf_counter() - t0, stride, gpu.get("c2_ms"),
          f"every {stride}th query row of 8192 (score, bf16 quantise, stable top-k)")
    c2 = out["C2"]
    del q, k, w

    # C3: every 8th row of 4096
    si = W.sfa_prefill_inputs(device="cuda:0", seed=42)
    q, k, qr, kr, idx = f(si.query), f(si.key), f(si.query_rope), f(si.key_rope), si.sparse_indices.cpu().numpy()
    scale = si.scale_value
    del si
    rows = [(0, s) for s in range(4095, -1, -8)]
    t0 = time.perf_counter()
    SFAO.sfa_golden_bsnd(q, k, idx, qr, kr, scale, [4096], [4096], 1, 3, "bf16", rows=rows)
    entry("C3", len(rows), 4096, time.perf_counter() - t0, 8, gpu.get("c3_ms"),
          "every 8th query row of 4096 (gather, scores, softmax, P@V)")
    del q, k, qr, kr, idx

    # C4: all 64 decode rows; each batch's pages de-paged on the host as the reference does
    sd = W.sfa_decode_inputs(device="cuda:0", seed=42)
    q, qr, kc, krc = f(sd.query), f(sd.query_rope), f(sd.key), f(sd.key_rope)
    idx, bt = sd.sparse_indices.cpu().numpy(), sd.block_table.cpu().numpy()
    lens, scale, bs = sd.actual_seq_lengths_kv, sd.scale_value, sd.block_size
    del sd
    t0 = time.perf_counter()
    for b in range(64):
        SFAO.sparse_flash_attention(q[b:b + 1], kc, None, idx[b:b + 1], scale, bt[b:b + 1], None, [lens[b]],
                                    qr[b:b + 1], krc, 1, "BSND", "PA_BSND", 3, True, block_size=bs,
                                    io_dtype="bf16")
    entry("C4", 64, 64, time.perf_counter() - t0, 1, gpu.get("c4_ms"),
          "all 64 rows (de-page each batch's cache, gather 2048 tokens, attention)")
    del q, qr, kc, krc

    # C5: every 16th row of each packed sequence, indexer then attention on its indices
    inp = W.tnd_pipeline_inputs(device="cuda:0", seed=42)
    cu = [0] + inp["cu_seqlens"].tolist()
    iq, ik, iw = f(inp["index_query"]), f(inp["index_key"]), f(inp["index_weights"])
    q, k, qr, kr = f(inp["query"]), f(inp["key"]), f(inp["query_rope"]), f(inp["key_rope"])
    scale, count = inp["scale_value"], inp["sparse_count"]
    del inp
    n_rows = 0
    t0 = time.perf_counter()
    for b in range(len(cu) - 1):
        a, e = cu[b], cu[b + 1]
        L = e - a
        rows = [(0, s) for s in range(L - 1, -1, -16)]
        n_rows += len(rows)
        ix, _ = LIO.li_golden_bsnd(iq[None, a:e], ik[None, a:e], iw[None, a:e], [L], [L], count, 3, False,
                                   rows=rows)
        SFAO.sfa_golden_bsnd(q[None, a:e], k[None, a:e], ix, qr[None, a:e], kr[None, a:e], scale,
                             [L], [L], 1, 3, "bf16", rows=rows)
    entry("C5", n_rows, cu[-1], time.perf_counter() - t0, 16, gpu.get("c5_ms"),
          "every 16th row of each of the 4 packed sequences (indexer, top-k, then attention on its indices)")
    return c2, out


def bench_indexer_c2(args, torch, W, dsa):
    from dsa_triton_ascend_amd.lightning_indexer import IndexerPlan
    dev = torch.device("cuda:0")
    c = dict(W.C2)
    inp = W.indexer_inputs(**c, device=dev, seed=42)
    plan = IndexerPlan(inp.query, inp.key, inp.weights, sparse_count=c["sparse_count"],
                       sparse_mode=3, return_value=True)
    warm(plan.run, torch)
    sec = timed(plan.run, args.steps, args.warmup, torch)
    t_score, t_topk = event_time([plan.score, plan.topk], max(10, args.steps), torch)
    # the public entry point: validation, output / score-scratch allocation and the small
    # host-to-device length copies on every call, as a caller without a plan pays them
    public = lambda: dsa.lightning_indexer(inp.query, inp.key, inp.weights, sparse_count=c["sparse_count"],
                                           sparse_mode=3, return_value=True)
    warm(public, torch)
    sec_public = timed(public, args.steps, 2, torch)
    S = c["S1"]
    pairs = S * (S + 1) // 2
    flop = 2.0 * pairs * c["N1"] * c["D"]
    return inp, c, sec, t_score, t_topk, flop, sec_public


def bench_sfa(plan_kwargs, steps, warmup, torch):
    from dsa_triton_ascend_amd.sparse_flash_attention import AttentionPlan
    plan = AttentionPlan(**plan_kwargs)
    warm(plan.run, torch)
    sec = timed(plan.run, steps, warmup, torch)
    (ms,) = event_time([plan.run], steps, torch)
    return sec, ms


# C5 algorithmic work (four causal sequences 1024/3000/6000/8192, top-2048):
# indexer sum_b L_b (L_b + 1) / 2 = 56,587,828 visible pairs x 64 heads x 128 x 2;
# attention sum_b sum_s min(s + 1, 2048) = 29,445,632 (row, token) pairs x 128 heads
# x (576 + 512) x 2.
C5_LI_FLOP = 56587828 * 64 * 128 * 2.0
C5_SFA_FLOP = 29445632 * 128 * (576 + 512) * 2.0


def bench_pipeline_c5(W, reps, torch):
    """End-to-end C5 rows/s (indexer score + top-k + SFA, one stream, no host sync)
    and the per-stage device times."""
    from dsa_triton_ascend_amd.pipeline import PrefillPlan
    inp = W.tnd_pipeline_inputs(device="cuda:0", seed=42)
    cu = inp["cu_seqlens"].tolist()
    plan = PrefillPlan(inp["index_query"], inp["index_key"], inp["index_weights"], inp["query"],
                       inp["key"], inp["query_rope"], inp["key_rope"], cu,
                       sparse_count=inp["sparse_count"], scale_value=inp["scale_value"])
    rows = int(cu[-1])
    warm(plan.run, torch)
    (t_all,) = event_time([plan.run], reps, torch)
    t_score, t_topk, t_sfa = event_time([plan.indexer.score, plan.indexer.topk, plan.attention.run], reps, torch)
    res = {"ms": round(t_all, 4), "rows_per_s": round(rows / (t_all * 1e-3), 1), "rows": rows,
           "li_score_ms": round(t_score, 4), "li_topk_ms": round(t_topk, 4), "sfa_ms": round(t_sfa, 4),
           "li_tflops": round(C5_LI_FLOP / t_score / 1e9, 2), "sfa_tflops": round(C5_SFA_FLOP / t_sfa / 1e9, 2),
           "sfa_frac_mfma": round(C5_SFA_FLOP / t_sfa / 1e9 / PEAK_BF16_TFLOPS, 4)}
    del plan, inp
    return res


def bench_grad(W, torch):
    """sparse_flash_attention_grad at perf_sfa_grad_triton.py:23's shape (the reference
    quotes 34 ms for it on Ascend 910, docs/sfa_grad_optimization_summary.md:9).
    Algorithmic work: 512 rows x 2048 tokens x 64 heads x 2 (3 x 576 + 2 x 512) FLOP."""
    from dsa_triton_ascend_amd import sparse_flash_attention
    from dsa_triton_ascend_amd.sparse_flash_attention_grad import GradPlan
    g = W.sfa_grad_inputs(device="cuda:0", seed=42, **W.GRAD_PERF)
    out, smax, ssum = sparse_flash_attention(g.query, g.key, g.key, g.sparse_indices, **g.kwargs())
    plan = GradPlan(g.query, g.key, g.key, g.sparse_indices, g.extra["d_out"], out, smax, ssum,
                    scale_value=g.scale_value, query_rope=g.query_rope, key_rope=g.key_rope,
                    sparse_mode=g.sparse_mode)
    warm(plan.run, torch)
    (ms,) = event_time([plan.run], 10, torch)
    flop = GRAD_PAIRS * 64 * 2.0 * (3 * 576 + 2 * 512)
    res = {"ms": round(ms, 4), "tflops": round(flop / ms / 1e9, 2),
           "frac_mfma": round(flop / ms / 1e9 / PEAK_BF16_TFLOPS, 4), "algorithmic_flop": flop,
           "shape": "BSND B=1 S1=512 S2=4096 N1=64 D=512+64 top-k 2048 causal bf16"}
    del plan, g, out, smax, ssum
    return res


# every row of the grad perf shape sees >= 3585 keys, so all select 2048 tokens
GRAD_PAIRS = 512 * 2048


def bench_kl(W, torch):
    """sparse_lightning_indexer_grad_kl_loss at the reference's target shape
    (test_sli_grad_kl_loss_triton.py:27: B=1, S1=512, S2=4096, N1=64, D=512 + 64 rope,
    Nidx1=64, D_idx=128, top-k 2048; every row uses 2048 slots). Algorithmic work per
    slot: teacher 64 x 576 x 2, student I, dQI and dKI 3 x 64 x 128 x 2 FLOP."""
    from dsa_triton_ascend_amd import sparse_flash_attention
    from dsa_triton_ascend_amd.sli_grad_kl_loss import KLLossPlan
    g = W.sfa_grad_inputs(device="cuda:0", seed=42, **W.GRAD_PERF)
    gen = torch.Generator(device="cuda:0").manual_seed(5)
    qi = torch.randn(1, 512, 64, 128, device="cuda:0", generator=gen).to(torch.bfloat16)
    ki = torch.randn(1, 4096, 1, 128, device="cuda:0", generator=gen).to(torch.bfloat16)
    w = torch.rand(1, 512, 64, device="cuda:0", generator=gen).to(torch.bfloat16)
    _, smax, ssum = sparse_flash_attention(g.query, g.key, g.key, g.sparse_indices, **g.kwargs())
    plan = KLLossPlan(g.query, g.key, qi, ki, w, g.sparse_indices, smax, ssum, query_rope=g.query_rope,
                      key_rope=g.key_rope, scale_value=g.scale_value)
    warm(plan.run, torch)
    (ms,) = event_time([plan.run], 10, torch)
    flop = 512 * 2048 * 2.0 * (64 * 576 + 3 * 64 * 128)
    res = {"ms": round(ms, 4), "tflops": round(flop / ms / 1e9, 2),
           "frac_mfma": round(flop / ms / 1e9 / PEAK_BF16_TFLOPS, 4), "algorithmic_flop": flop,
           "shape": "BSND B=1 S1=512 S2=4096 N1=64 D=512+64 Nidx1=64 D_idx=128 top-k 2048 bf16"}
    del plan, g, qi, ki, w
    return res


def bench_dense(torch):
    """Dense indexer loss at the reference's perf shape (perf_dense_loss_backward_triton.py:18:
    B=1, S1=512, S2=4096, N1=N2=64, D=128 + 64 rope, Nidx1=64, D_idx=128, fp16): the
    softmax LSE, then the loss backward with those stats. Every row s1 sees
    4096 - 512 + s1 + 1 keys; algorithmic work per key: LSE 64 x 128 x 2, loss teacher
    64 x 192 x 2 plus student I, dQI and dKI 3 x 64 x 128 x 2 FLOP."""
    from dsa_triton_ascend_amd.dense_loss import DenseLossPlan, dense_lightning_indexer_softmax_lse
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(11)
    r = lambda *s: torch.randn(*s, device=dev, generator=gen).to(torch.float16)
    B, S1, S2, N1, D, Nidx1, Didx = 1, 512, 4096, 64, 128, 64, 128
    q, k, qr, kr = r(B, S1, N1, D), r(B, S2, N1, D), r(B, S1, N1, 64), r(B, S2, N1, 64)
    qi, ki = r(B, S1, Nidx1, Didx), r(B, S2, 1, Didx)
    w = torch.rand(B, S1, Nidx1, device=dev, generator=gen).to(torch.float16)
    smax = torch.zeros(B, N1, S1, 1, device=dev)
    ssum = torch.full((B, N1, S1, 1), 64.0, device=dev)
    lse = lambda: dense_lightning_indexer_softmax_lse(qi, ki, w)
    mxi, smi = lse()
    plan = DenseLossPlan(q, k, qi, ki, w, smax, ssum, mxi, smi, 1.0 / 192 ** 0.5, qr, kr)
    warm(plan.run, torch)
    warm(lse, torch)
    ms_lse, ms = event_time([lse, plan.run], 10, torch)
    keys = sum(S2 - S1 + s1 + 1 for s1 in range(S1))
    f_lse = keys * 64 * 128 * 2.0
    f_loss = keys * 2.0 * (64 * 192 + 3 * 64 * 128)
    res = {"lse_ms": round(ms_lse, 4), "lse_tflops": round(f_lse / ms_lse / 1e9, 2),
           "loss_ms": round(ms, 4), "loss_tflops": round(f_loss / ms / 1e9, 2),
           "frac_mfma": round(f_loss / ms / 1e9 / PEAK_BF16_TFLOPS, 4), "algorithmic_flop": f_loss,
           "shape": "BSND B=1 S1=512 S2=4096 N1=N2=64 D=128+64 Nidx1=64 D_idx=128 fp16"}
    del plan, q, k, qr, kr, qi, ki, w
    return res


def pmc_pass(torch, W):
    from dsa_triton_ascend_amd.lightning_indexer import IndexerPlan
    from dsa_triton_ascend_amd.sparse_flash_attention import AttentionPlan
    dev = torch.device("cuda:0")
    src = torch.empty(256 << 20, dtype=torch.bfloat16, device=dev).fill_(1.0)   # 512 MiB
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)                                      # calibration: reads and writes 512 MiB
    torch.cuda.synchronize()
    del src, dst
    c = dict(W.C2)
    inp = W.indexer_inputs(**c, device=dev, seed=42)
    plan = IndexerPlan(inp.query, inp.key, inp.weights, sparse_count=c["sparse_count"], sparse_mode=3,
                       return_value=True)
    plan.run()
    torch.cuda.synchronize()
    del plan, inp
    li = W.indexer_inputs(B=1, S1=512, S2=4096, N1=64, N2=1, D=128, sparse_count=2048, sparse_mode=3,
                          w_scale=1.0, dtype=torch.float16, device=dev, seed=42)   # perf_li shape
    IndexerPlan(li.query, li.key, li.weights, sparse_count=2048, sparse_mode=3, return_value=True).run()
    torch.cuda.synchronize()
    del li
    for mk in (W.sfa_prefill_inputs, W.sfa_decode_inputs):
        si = mk(device="cuda:0", seed=42)
        AttentionPlan(query=si.query, key=si.key, value=si.key, sparse_indices=si.sparse_indices,
                      **si.kwargs()).run()
        torch.cuda.synchronize()
        del si
    from dsa_triton_ascend_amd import sparse_flash_attention
    from dsa_triton_ascend_amd.sparse_flash_attention_grad import GradPlan
    g = W.sfa_grad_inputs(device="cuda:0", seed=42, **W.GRAD_PERF)
    out, smax, ssum = sparse_flash_attention(g.query, g.key, g.key, g.sparse_indices, **g.kwargs())
    GradPlan(g.query, g.key, g.key, g.sparse_indices, g.extra["d_out"], out, smax, ssum,
             scale_value=g.scale_value, query_rope=g.query_rope, key_rope=g.key_rope,
             sparse_mode=g.sparse_mode).run()
    torch.cuda.synchronize()
    log("[pmc-pass] done")


def committed_traffic(kernel):
    """HBM bytes per launch measured by the rocprofv3 FETCH_SIZE / WRITE_SIZE passes
    (profiles/pmc_traffic.json, written from those runs), scaled by the copy calibration."""
    path = os.path.join(ROOT, "profiles", "pmc_traffic.json")
    try:
        with open(path) as f:
            d = json.load(f)
        return d["kernels"][kernel]["hbm_bytes_per_launch"]
    except Exception:
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--quick", action="store_true", help="headline only (no breakdown, no CPU baseline)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="for rocprofv3 --pmc: one C2 indexer call, one SFA prefill/decode call and a "
                         "512 MiB plain copy (the counter calibration), no timing")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    import dsa_triton_ascend_amd as dsa
    from dsa_triton_ascend_amd import workloads as W

    if args.pmc_pass:
        pmc_pass(torch, W)
        return

    log("[bench] C2 lightning_indexer ...")
    inp, c, sec, t_score, t_topk, flop, sec_public = bench_indexer_c2(args, torch, W, dsa)
    del inp
    rows = c["S1"]
    achieved = flop / (t_score * 1e-3) / 1e12
    result = {
        "metric": METRIC,
        "value": round(rows / sec, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 inputs of the BASELINE config shapes)",
        "config": {"workload": "C2: lightning_indexer BSND B=1 S1=S2=8192 N1=64 N2=1 D=128 "
                               "sparse_count=2048 sparse_mode=3 return_value=True",
                   "rows": rows, "indexer_tflops": round(flop / sec / 1e12, 2),
                   "public_call_ms": round(sec_public * 1e3, 4),
                   "public_call_note": "lightning_indexer() itself: validation, output and score-scratch "
                                       "allocation, length copies; value / ms_per_step time IndexerPlan.run"},
        "roofline": {"kernel": "li_score_kernel", "bound": "mfma", "achieved": round(achieved, 2),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": committed_traffic("li_score_kernel"), "kernel_ms": round(t_score, 4),
                     "algorithmic_flop": flop},
    }
    breakdown = {"li_topk_kernel_ms": round(t_topk, 4),
                 "li_topk_rows_per_s": round(rows / (t_topk * 1e-3), 1)}
    gpu_ms = {"c2_ms": sec * 1e3}
    if not args.quick:
        log("[bench] C1 lightning_indexer ...")
        from dsa_triton_ascend_amd.lightning_indexer import IndexerPlan
        i1 = W.indexer_inputs(**W.C1, device="cuda:0", seed=42)
        p1 = IndexerPlan(i1.query, i1.key, i1.weights, sparse_count=64, sparse_mode=3, return_value=True)
        warm(p1.run, torch)
        (gpu_ms["c1_ms"],) = event_time([p1.run], 50, torch)
        breakdown["indexer_c1"] = {"ms": round(gpu_ms["c1_ms"], 4),
                                   "rows_per_s": round(256 / (gpu_ms["c1_ms"] * 1e-3), 1)}
        del p1, i1
        log("[bench] lightning_indexer at the reference's perf_li shape ...")
        # perf_li_triton.py:43: B=1, S1=512, S2=4096, N1=64, N2=1, D=128, top-k 2048, fp16
        # inputs, fp32 weights N(0,1), the cell's default causal mode 3
        ip = W.indexer_inputs(B=1, S1=512, S2=4096, N1=64, N2=1, D=128, sparse_count=2048, sparse_mode=3,
                              w_scale=1.0, dtype=torch.float16, device="cuda:0", seed=42)
        pp = IndexerPlan(ip.query, ip.key, ip.weights, sparse_count=2048, sparse_mode=3, return_value=True)
        warm(pp.run, torch)
        ms_li, ms_li_score, ms_li_topk = event_time([pp.run, pp.score, pp.topk], 50, torch)
        pairs_li = sum(4096 - 512 + s + 1 for s in range(512))
        f_li = 2.0 * pairs_li * 64 * 128
        breakdown["indexer_perf_li"] = {"ms": round(ms_li, 4), "score_ms": round(ms_li_score, 4),
                                        "topk_ms": round(ms_li_topk, 4),
                                        "rows_per_s": round(512 / (ms_li * 1e-3), 1),
                                        "score_tflops": round(f_li / ms_li_score / 1e9, 2),
                                        "score_frac_mfma": round(f_li / ms_li_score / 1e9 / PEAK_BF16_TFLOPS, 4),
                                        "algorithmic_flop": f_li,
                                        "shape": "BSND B=1 S1=512 S2=4096 N1=64 N2=1 D=128 top-k 2048 causal fp16 "
                                                 "(perf_li_triton.py:43)"}
        del pp, ip
        steps = max(3, args.steps // 4)
        try:
            log("[bench] C3 SFA prefill ...")
            si = W.sfa_prefill_inputs(device="cuda:0", seed=42)
            kw = dict(query=si.query, key=si.key, value=si.key, sparse_indices=si.sparse_indices, **si.kwargs())
            s3, ms3 = bench_sfa(kw, 10, 1, torch)
            f3 = 6292480 * 128 * (576 + 512) * 2.0
            gpu_ms["c3_ms"] = ms3
            breakdown["sfa_prefill_c3"] = {"ms": round(ms3, 4), "tflops": round(f3 / ms3 / 1e9, 2),
                                           "frac_mfma": round(f3 / ms3 / 1e9 / PEAK_BF16_TFLOPS, 4),
                                           "algorithmic_flop": f3}
            del si, kw
            torch.cuda.empty_cache()
            log("[bench] C4 SFA decode ...")
            sd = W.sfa_decode_inputs(device="cuda:0", seed=42)
            kw = dict(query=sd.query, key=sd.key, value=sd.key, sparse_indices=sd.sparse_indices, **sd.kwargs())
            s4, ms4 = bench_sfa(kw, 50, 2, torch)
            kv_bytes = 64 * 2048 * 576 * 2
            gpu_ms["c4_ms"] = ms4
            breakdown["sfa_decode_c4"] = {"ms": round(ms4, 4), "kv_gbs": round(kv_bytes / ms4 / 1e6, 1),
                                          "frac_hbm": round(kv_bytes / ms4 / 1e6 / PEAK_HBM_GBS, 4),
                                          "gathered_kv_bytes": kv_bytes}
            del sd, kw
            torch.cuda.empty_cache()
            log("[bench] SFA prefill at the reference's perf_sfa shape (N1=64) ...")
            sg = W.sfa_grad_inputs(device="cuda:0", seed=42, **W.GRAD_PERF)
            kw = dict(query=sg.query, key=sg.key, value=sg.key, sparse_indices=sg.sparse_indices, **sg.kwargs())
            _, ms64 = bench_sfa(kw, 20, 1, torch)
            f64 = GRAD_PAIRS * 64 * (576 + 512) * 2.0
            breakdown["sfa_prefill_n64"] = {"ms": round(ms64, 4), "tflops": round(f64 / ms64 / 1e9, 2),
                                            "frac_mfma": round(f64 / ms64 / 1e9 / PEAK_BF16_TFLOPS, 4),
                                            "algorithmic_flop": f64,
                                            "shape": "BSND B=1 S1=512 S2=4096 N1=64 D=512+64 top-k 2048 causal bf16 "
                                                     "(perf_sfa_triton.py:7-9)"}
            del sg, kw
            torch.cuda.empty_cache()
            log("[bench] SFA backward at the reference's grad perf shape ...")
            breakdown["sfa_grad"] = bench_grad(W, torch)
            torch.cuda.empty_cache()
            log("[bench] sparse LI grad KL loss at the reference's target shape ...")
            breakdown["sli_grad_kl_loss"] = bench_kl(W, torch)
            breakdown["dense_li_loss"] = bench_dense(torch)
            torch.cuda.empty_cache()
            log("[bench] C5 TND indexer -> SFA pipeline ...")
            breakdown["pipeline_c5"] = bench_pipeline_c5(W, max(3, args.steps // 4), torch)
            gpu_ms["c5_ms"] = breakdown["pipeline_c5"]["ms"]
            torch.cuda.empty_cache()
        except Exception as e:  # report, keep the headline
            breakdown["sfa_error"] = repr(e)[:300]
    if not (args.quick or args.no_cpu):
        log("[bench] CPU baseline (numpy oracle on this host: C1, C4 in full; C2, C3, C5 sampled) ...")
        cores, model, blas = cpu_host_info()
        c2, per_cfg = cpu_baselines(torch, W, gpu_ms)
        result["cpu_baseline"] = {
            "value": c2["cpu_rows_per_s"], "unit": "rows/s", "cores": cores, "kind": "port",
            "sample": f"C2: {c2['rows_sampled']} of 8192 query rows (every {c2['stride']}th, spanning the "
                      f"causal triangle) through the numpy oracle (score, bf16 quantise, stable top-k); "
                      f"{c2['cpu_s']} s; full call extrapolates to {c2['extrapolated_full_call_s']} s",
            "cpu_model": model, "blas_threads": blas,
            "cores_note": "len(os.sched_getaffinity(0)); numpy BLAS threads as listed",
            "configs": per_cfg}
    else:
        result["cpu_baseline"] = None
    result["breakdown"] = breakdown
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
