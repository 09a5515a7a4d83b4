#!/usr/bin/env python3
"""Benchmark of the MI355X verify path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Prints ONE JSON line (rank 0). Workloads:
  spec    - (default) config 3: speculative decoding at batch 1, random-init
            Qwen3-8B target (36 layers, hidden 4096, 32/8 heads, FFN 12288,
            V 151936) and Qwen3-0.6B draft (28 layers, hidden 1024, 16/8 heads,
            FFN 3072), gamma 3, 64-token prompt, T=0.6, reference acceptance.
            One step = draft phase (pre-allocation + 3 draft tokens) + verify
            phase (target forward over 4 tokens, LM head, fused acceptance,
            commit), each replayed as a HIP graph. value = emitted tokens per
            second of GPU time over the timed steps; verify_accept_step_us is
            the verify-phase time per step.
  accept  - the fused acceptance op alone (one hs_spec_accept call per step).
            Defaults: the batch-1 verify shape of the spec run (B=1, gamma=3,
            bf16 target logits, f32 draft probabilities, T=0.6, reference
            acceptance). --batch/--gamma/--mode/--logits/--per-seq select the
            other sampler shapes (config 0: --logits f32 --mode filtered
            --temperature 1 --top-k 50 --top-p 0.9; config 1: --batch 8|64|256
            --gamma 1|3|5 --per-seq --mode filtered, or --mode greedy).
  gemm    - the spec step's dominant kernel alone: the 8B target's gate/up
            projection at the verify shape over 36 weight sets.
  attention - config 2: paged verify attention, B=64, 4 queries, 16 Q / 8 KV
            heads, D=128, context ~ U[64, 2048], 256-token blocks in a random
            permutation, bf16 or (--kv fp8) fp8-e4m3 cache.
Timed launches are captured in HIP graphs and replayed between two HIP events
on the launch stream; inputs rotate over enough copies that every step reads
HBM (the MI355X MALL is 256 MB).
The roofline figure is algorithmic bytes per launch of the workload's dominant
kernel divided by its HIP-event time measured on the launch stream. spec: the
verify-attention launch the step runs once per layer (hs_qk_norm_rope_attend:
q/k-norm + RoPE of the 4 qkv rows, their K/V stored, then the attention) at the
batch-1 verify shape with context 320 (64 prompt + 256 generated tokens);
roofline_inscope_step is the verify+accept step's own work (36 such launches,
the acceptance with the step's bookkeeping in one launch) against its bytes,
without the projection weights; roofline_gemm is the gate/up projection of the target (the
largest share of the step's kernel time, a weight stream) and roofline_step the
whole verify phase against the weights it streams. accept and attention: the
whole call. cpu_baseline times the torch-CPU restatement of the reference loop
(oracle/torch_port.py) on the host cores of the same machine on a bounded sample.
"""
from __future__ import annotations

import argparse
import importlib
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "verify+accept step µs and accepted tok/s @B=1 γ=3 (8B tgt/0.6B draft)"
HBM_PEAK_GBS = 8000.0
V = 151936


def graph_time_us(torch, dev, fn, reps: int) -> float:
    """Capture fn() (a fixed sequence of launches) as one HIP graph and return the
    GPU time of one replay in µs, averaged over `reps` replays timed with HIP events
    on the launch stream."""
    fn()  # eager call first: creates every workspace outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            fn()
    torch.cuda.current_stream(dev).wait_stream(s)
    graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps


def _accept_inputs(torch, hv, dev, args):
    """Sampler inputs generated on the device: target logits ~ N(0, 2^2), draft
    logits = target[:, :gamma] + N(0, 1); the draft probabilities and tokens are the
    draft distribution (filtered in filtered mode) and a draw from it."""
    B, g = args.batch, args.gamma
    gen = torch.Generator(device=dev).manual_seed(0)
    target = torch.randn((B, g + 1, V), generator=gen, device=dev) * 2.0
    draft = target[:, :g] + torch.randn((B, g, V), generator=gen, device=dev)
    if args.logits == "bf16":
        target = target.to(torch.bfloat16)
        draft = draft.to(torch.bfloat16)
    if args.per_seq:
        temps = torch.rand(B, generator=gen, device=dev) * 0.7 + 0.5
        choice = torch.randint(0, 3, (2, B), generator=gen, device=dev)
        top_ks = torch.tensor([0, 20, 50], device=dev, dtype=torch.int32)[choice[0]]
        top_ps = torch.tensor([1.0, 0.9, 0.8], device=dev)[choice[1]]
    else:
        temps = torch.full((B,), args.temperature, device=dev)
        top_ks = torch.full((B,), args.top_k, device=dev, dtype=torch.int32)
        top_ps = torch.full((B,), args.top_p, device=dev)
    u = torch.rand(B * g, generator=gen, device=dev)
    if args.mode == "greedy":
        q, dtok = None, draft.float().argmax(-1)
    else:
        rows = draft.reshape(B * g, V)
        r = hv.ops.sample_rows(rows, temps.repeat_interleave(g), top_ks.repeat_interleave(g),
                               top_ps.repeat_interleave(g), mode=args.mode, uniforms=u,
                               want_probs=True)
        q, dtok = r["probs"].view(B, g, V), r["tokens"].view(B, g)
    small = dict(draft_tokens=dtok, temperatures=temps, top_ks=top_ks, top_ps=top_ps,
                 u_accept=torch.rand((B, g), generator=gen, device=dev),
                 u_resample=torch.rand(B, generator=gen, device=dev))
    return target, q, small


def _topk_hint(args) -> bool:
    """The caller-side promise that every top-k is in [1, 64] (the single top-k
    launch for small batches)."""
    return (args.mode == "filtered" and not args.per_seq and 1 <= args.top_k <= 64
            and not args.no_topk_hint)


def _accept_valu_busy(tag: str):
    """VALU-busy percentage of the acceptance call's longest-running profiled kernel
    (the single launch, or the chain's row-statistics / filter passes)."""
    for k in ("k_accept_small_topk<float, 3>", "k_accept_small<bf16, 3>",
              "k_chunk_stats_w<bf16>", "k_filter_pass1_kp<bf16>", "k_filter_pass1<float>",
              "k_filter_pass1<bf16>"):
        v = profiled_counter(k, tag, "VALUBusy %")
        if v is not None:
            return v
    return None


def _accept_tag(args) -> str:
    tag = f"accept-b{args.batch}-g{args.gamma}-{args.mode}-{args.logits}"
    return tag + ("-perseq" if args.per_seq else "") + ("-topk" if _topk_hint(args) else "")


def bench_accept(args, torch, hv):
    dev = torch.device("cuda:0")
    B, gamma = args.batch, args.gamma
    esz = 2 if args.logits == "bf16" else 4
    # algorithmic bytes: every target row once, plus the draft rows in the sampling modes
    step_bytes = B * (gamma + 1) * V * esz + (0 if args.mode == "greedy" else B * gamma * V * 4)
    copies = max(2, int(512e6 // step_bytes) + 1)
    target, q, s = _accept_inputs(torch, hv, dev, args)
    bufs = [(target.clone(), None if q is None else q.clone()) for _ in range(copies)]
    del target, q

    topk_le64 = _topk_hint(args)

    def step(i):
        lg, qq = bufs[i % copies]
        return hv.ops.spec_accept(lg, qq, s["draft_tokens"], s["temperatures"], s["u_accept"],
                                  s["u_resample"], mode=args.mode, top_ks=s["top_ks"],
                                  top_ps=s["top_ps"], topk_le64=topk_le64,
                                  chain_only=args.chain)

    outs = []

    def one_round():
        outs.clear()
        for i in range(copies):
            outs.append(step(i))

    reps_w = max(1, -(-args.warmup // copies))
    reps = max(1, -(-args.steps // copies))
    graph_time_us(torch, dev, one_round, reps_w)  # warm-up replays
    t0 = time.perf_counter()
    us_round = graph_time_us(torch, dev, one_round, reps)
    wall = time.perf_counter() - t0
    us_per_step = us_round / copies
    steps = reps * copies
    nacc = outs[-1][0].cpu().tolist()
    achieved = step_bytes / (us_per_step * 1e-6) / 1e9
    shape = f"B={B} gamma={gamma} V={V} {args.logits} logits, mode {args.mode}"
    res = {
        "metric": METRIC,
        "value": round(us_per_step, 3),
        "unit": "us/step (fused acceptance)",
        "n_gpus": 1,
        "steps": steps,
        "warmup": reps_w * copies,
        "ms_per_step": round(us_per_step / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"{args.logits} logits, f32 math",
        "data": "synthetic (seeded N(0,2^2) logits, draft = target + N(0,1))",
        "config": {"workload": f"fused acceptance, {shape}", "batch": B, "gamma": gamma,
                   "vocab": V, "mode": args.mode,
                   "sampling": "per-seq T~U[0.5,1.2], top-k {0,20,50}, top-p {1,0.9,0.8}"
                   if args.per_seq else f"T={args.temperature} top-k={args.top_k} top-p={args.top_p}",
                   "input_copies_rotated": copies, "topk_le64": topk_le64,
                   "chain_only": bool(args.chain)},
        "accepted_mean": round(sum(nacc) / len(nacc), 3),
        "wall_s": round(wall, 3),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic("hs_spec_accept call", _accept_tag(args)),
                     "mfma_util": 0.0,
                     "valu_busy": _accept_valu_busy(_accept_tag(args)),
                     "bytes_per_step": step_bytes,
                     "kernels": "one hs_spec_accept call: k_accept_small for reference-mode "
                                "calls that fit one workgroup per CU, k_accept_small_topk "
                                "for such filtered calls with every top-k in [1, 64], else "
                                "the chain (row statistics, filter when filtered, decision + "
                                "resample partials, final search)"},
    }
    if not args.no_cpu_baseline:
        # one sequence of the same settings (the per-sequence settings of a batch
        # vary; its first sequence's are used)
        if args.per_seq or args.mode == "greedy":
            w = hv.synthetic.accept_workload(1, gamma, seed=0, dtype=args.logits,
                                             temperature=0.6)
            mode = "reference"
        else:
            w = hv.synthetic.accept_workload(1, gamma, seed=0, dtype=args.logits,
                                             temperature=args.temperature, top_k=args.top_k,
                                             top_p=args.top_p, mode=args.mode)
            mode = args.mode
        res["cpu_baseline"] = cpu_baseline_accept(torch, w, args.cpu_seconds, mode=mode,
                                                  logits=args.logits)
    return res


def bench_sampler(args, torch, hv):
    """The draft step's row sampler alone (model_runner.py:312-313 with
    sampler.py:13-25): softmax(logits / T) of --batch rows written into one column of
    a [B, 3, V] draft-probability buffer (as the draft phase writes it) and one token
    per row drawn with an explicit uniform; --logits bf16 (default) or f32 ~ N(0, 2^2),
    T = --temperature, reference mode (a few rows run as one launch; --chain forces the
    launch chain). Inputs rotate over copies so every call reads HBM."""
    dev = torch.device("cuda:0")
    B = args.batch
    esz = 2 if args.logits == "bf16" else 4
    step_bytes = B * V * esz + B * V * 4 + B * 8  # logits read, probabilities and tokens written
    copies = max(2, int(512e6 // (B * V * esz)) + 1)
    gen = torch.Generator(device=dev).manual_seed(0)
    lg = torch.randn((B, V), generator=gen, device=dev) * 2.0
    if args.logits == "bf16":
        lg = lg.to(torch.bfloat16)
    bufs = [lg.clone() for _ in range(copies)]
    del lg
    probs = torch.empty((B, 3, V), dtype=torch.float32, device=dev)
    toks = torch.empty(B, dtype=torch.int64, device=dev)
    temps = torch.full((B,), args.temperature, device=dev)
    u = torch.rand(B, generator=gen, device=dev)

    def one_round():
        for i in range(copies):
            hv.ops.sample_rows(bufs[i], temps, mode="reference", uniforms=u,
                               probs_out=probs[:, 1], tokens_out=toks, chain_only=args.chain)

    reps_w = max(1, -(-args.warmup // copies))
    reps = max(1, -(-args.steps // copies))
    graph_time_us(torch, dev, one_round, reps_w)
    us = graph_time_us(torch, dev, one_round, reps) / copies
    achieved = step_bytes / (us * 1e-6) / 1e9
    tag = f"sampler-b{B}-{args.logits}" + ("-chain" if args.chain else "")
    kernel = "k_sample_small<bf16>" if args.logits == "bf16" else "k_sample_small<float>"
    return {"metric": METRIC, "value": round(us, 3), "unit": "us/call (row sampler)",
            "n_gpus": 1, "steps": reps * copies, "warmup": reps_w * copies,
            "ms_per_step": round(us / 1e3, 6), "higher_is_better": False, "scaling": "weak",
            "vs_baseline": None, "dtype": f"{args.logits} logits, f32 math",
            "data": "synthetic (seeded N(0,2^2) logits)",
            "config": {"workload": f"draft-step row sampler, B={B} V={V} {args.logits}, "
                                   f"T={args.temperature}, reference mode",
                       "chain_only": bool(args.chain), "input_copies_rotated": copies},
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 5),
                         "traffic": None if args.chain else profiled_traffic(kernel, tag),
                         "bytes_per_step": step_bytes,
                         "kernels": "one hs_sampler call: k_sample_small for a few rows, "
                                    "else the chain (chunk statistics, probabilities and "
                                    "partial sums, final search)"}}


def bench_attention(args, torch, hv):
    """Config 2: B=64 sequences x 4 verify queries, 16/8 heads, D=128, L ~ U[64, 2048],
    256-token blocks in a random permutation; bf16 or fp8-e4m3 cache."""
    import numpy as np
    dev = torch.device("cuda:0")
    B, R, Hq, Hkv, D, bs = 64, 4, 16, 8, 128, 256
    rng = np.random.default_rng(0)
    lens = rng.integers(64, 2049, size=B)
    nblk = (lens + bs - 1) // bs
    nb = int(nblk.sum()) + 3
    perm = rng.permutation(nb).astype(np.int32)
    bt = np.full((B, int(nblk.max())), -1, np.int32)
    off = 0
    for b in range(B):
        bt[b, :nblk[b]] = perm[off:off + nblk[b]]
        off += nblk[b]
    fp8 = args.kv == "fp8"
    gen = torch.Generator(device=dev).manual_seed(0)
    kv_bytes_all = 2 * nb * bs * Hkv * D * (1 if fp8 else 2)
    copies = max(2, int(512e6 // kv_bytes_all) + 1)
    caches = []
    scale = 1.0
    for _ in range(copies):
        k = torch.randn((nb, bs, Hkv, D), generator=gen, device=dev)
        v = torch.randn((nb, bs, Hkv, D), generator=gen, device=dev)
        if fp8:
            scale = float(max(k.abs().max(), v.abs().max())) / 448.0
            k = (k / scale).to(torch.float8_e4m3fn)
            v = (v / scale).to(torch.float8_e4m3fn)
        else:
            k, v = k.to(torch.bfloat16), v.to(torch.bfloat16)
        caches.append((k, v))
    q = torch.randn((B * R, Hq, D), generator=gen, device=dev).to(torch.bfloat16)
    cu_q = torch.arange(0, B * R + 1, R, dtype=torch.int32, device=dev)
    cu_k = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=dev)
    btt = torch.from_numpy(bt).to(dev)
    maxk = int(lens.max())
    outs = [torch.empty((B * R, Hq, D), dtype=torch.bfloat16, device=dev) for _ in range(copies)]

    def one_round():
        for i, (k, v) in enumerate(caches):
            hv.ops.verify_attention(q, k, v, btt, cu_q, cu_k, R, maxk, D ** -0.5,
                                    k_scale=scale, v_scale=scale, out=outs[i])

    reps_w = max(1, -(-args.warmup // copies))
    reps = max(1, -(-args.steps // copies))
    graph_time_us(torch, dev, one_round, reps_w)
    t0 = time.perf_counter()
    us_round = graph_time_us(torch, dev, one_round, reps)
    wall = time.perf_counter() - t0
    us = us_round / copies
    kv_read = int(lens.sum()) * Hkv * D * 2 * (1 if fp8 else 2)
    per_launch = kv_read + 2 * (B * R * Hq * D * 2)
    achieved = per_launch / (us * 1e-6) / 1e9
    flops = 4 * int(lens.sum()) * R * Hq * D
    # a call this size runs as the balanced launch (one workgroup per CU, one kv head per wave)
    main_kernel = f"k_verify_attn_sk<{'true' if fp8 else 'false'}, 2, true>"
    res = {
        "metric": METRIC,
        "value": round(us, 3),
        "unit": "us/launch (verify attention)",
        "n_gpus": 1,
        "steps": reps * copies,
        "warmup": reps_w * copies,
        "ms_per_step": round(us / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8-e4m3 KV, bf16 MFMA" if fp8 else "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v, random block permutation)",
        "config": {"workload": "config 2: paged verify attention B=64 q=4 Hq=16 Hkv=8 D=128 "
                               "L~U[64,2048] block 256", "kv_cache": args.kv,
                   "mean_context": round(float(lens.mean()), 1), "input_copies_rotated": copies},
        "tflops": round(flops / (us * 1e-6) / 1e12, 3),
        "wall_s": round(wall, 3),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": call_traffic([main_kernel, "k_attn_combine_sk<true>"],
                                             f"attention-{args.kv}"),
                     "mfma_util": profiled_counter(main_kernel, f"attention-{args.kv}",
                                                   "MfmaUtil %"),
                     "bytes_per_launch": per_launch,
                     "kernel": f"{main_kernel} + k_attn_combine_sk<true> (one call, timed together)"},
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline_attention(torch, lens, bs, R, Hq, Hkv, D,
                                                     args.cpu_seconds)
    return res


def _host_cores():
    """(os.cpu_count(), nproc): the machine's logical CPUs and those this process
    may run on (its affinity mask, what `nproc` prints)."""
    n_os = os.cpu_count() or 1
    try:
        n_proc = len(os.sched_getaffinity(0))
    except AttributeError:
        n_proc = n_os
    return n_os, n_proc


def _timed_at_threads(torch, fn, threads: int, seconds: float, min_iters: int):
    torch.set_num_threads(threads)
    fn()
    n = 0
    t0 = time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds and n >= min_iters:
            break
    return el / n, n, el


def _cpu_legs(torch, fn, seconds: float, min_iters: int):
    """Times fn at every usable core (nproc threads), at os.cpu_count() threads when
    that differs, and at 1 thread; the fastest multi-thread leg is the baseline."""
    n_os, n_proc = _host_cores()
    legs = {}
    for th in sorted({n_proc, n_os} - {1}) or [1]:
        legs[th] = _timed_at_threads(torch, fn, th, seconds, min_iters)
    legs[1] = _timed_at_threads(torch, fn, 1, seconds, min_iters)
    best = min((k for k in legs if k != 1), key=lambda k: legs[k][0], default=1)
    torch.set_num_threads(n_proc)
    return legs, best, n_os, n_proc


def cpu_baseline_accept(torch, w, seconds: float, mode: str = "reference",
                        logits: str = "bf16"):
    from oracle import torch_port
    lg = torch.from_numpy(w["logits"])  # (bf16-rounded) values as f32
    if logits == "bf16":
        lg = lg.to(torch.bfloat16)
    q = torch.from_numpy(w["draft_probs"])
    dt = torch.from_numpy(w["draft_tokens"])
    T = torch.from_numpy(w["temperatures"])
    ua = torch.from_numpy(w["u_accept"])
    ur = torch.from_numpy(w["u_resample"])
    B, g = dt.shape

    def fn():
        torch_port.run_verify_accept(lg, q, dt, T, ua, ur, mode=mode, top_ks=w["top_ks"],
                                     top_ps=w["top_ps"])

    legs, best, n_os, n_proc = _cpu_legs(torch, fn, seconds, 5)
    per, n, el = legs[best]
    return {"value": round(per * 1e6, 1), "unit": "us/step (fused acceptance)",
            "cores": best, "kind": "port",
            "single_thread": {"value": round(legs[1][0] * 1e6, 1), "cores": 1},
            "threads_tried": {str(k): round(v[0] * 1e6, 1) for k, v in sorted(legs.items())},
            "os_cpu_count": n_os, "nproc": n_proc,
            "sample": f"{n} acceptance steps at B={B} gamma={g} V=151936, {mode} mode, "
                      f"{logits} logits, over {el:.1f} s per leg (torch-CPU restatement of "
                      "model_runner.py:391-428" +
                      (" with sampler.py:27-49's top-k / top-p" if mode == "filtered" else "") +
                      ")"}


def cpu_baseline_attention(torch, lens, block_size: int, R: int, Hq: int, Hkv: int, D: int,
                           seconds: float, sample_seqs: int = 8):
    """The config-2 paged verify attention restated in torch-CPU fp32
    (oracle/torch_port.paged_attention), timed on a bounded sample: the first
    `sample_seqs` sequences of the workload, scaled to the whole batch by their
    share of the key count."""
    from oracle import torch_port
    sl = [int(x) for x in lens[:sample_seqs]]
    nblk = [(x + block_size - 1) // block_size for x in sl]
    nb = sum(nblk)
    gen = torch.Generator().manual_seed(0)
    kc = torch.randn((nb, block_size, Hkv, D), generator=gen)
    vc = torch.randn((nb, block_size, Hkv, D), generator=gen)
    bt = torch.full((len(sl), max(nblk)), -1, dtype=torch.int32)
    off = 0
    for b, n in enumerate(nblk):
        bt[b, :n] = torch.arange(off, off + n, dtype=torch.int32)
        off += n
    q = torch.randn((len(sl) * R, Hq, D), generator=gen)
    cu_q = [R * b for b in range(len(sl) + 1)]
    cu_k = [0]
    for x in sl:
        cu_k.append(cu_k[-1] + x)
    scale = D ** -0.5

    def fn():
        torch_port.paged_attention(q, kc, vc, bt, cu_q, cu_k, scale)

    legs, best, n_os, n_proc = _cpu_legs(torch, fn, seconds, 3)
    per_sample, n, el = legs[best]
    share = sum(sl) / float(sum(int(x) for x in lens))
    return {"value": round(per_sample / share * 1e6, 1), "unit": "us/launch (verify attention)",
            "cores": best, "kind": "port",
            "single_thread": {"value": round(legs[1][0] / share * 1e6, 1), "cores": 1},
            "threads_tried": {str(k): round(v[0] / share * 1e6, 1)
                              for k, v in sorted(legs.items())},
            "os_cpu_count": n_os, "nproc": n_proc,
            "sample": f"{n} passes over {len(sl)} of the {len(lens)} sequences ({sum(sl)} of "
                      f"{int(sum(int(x) for x in lens))} keys, fp32) in {el:.1f} s, scaled by "
                      "the key share (torch-CPU restatement of attention.py:147-160)"}


def _spec_runner(torch, sr, target, draft, kv: str, max_model_len: int, need: int):
    """A batch-1 config-3 runner: the reference's max_model_len (benchmarks/bench.py:181
    uses 4096) sizes the block tables and every attention launch plan; 0 sizes them
    to the `need` tokens of the run."""
    return sr.SpecRunner(target, draft, batch=1, gamma=3,
                         max_model_len=max_model_len if max_model_len > 0 else need,
                         temperature=0.6, mode="reference", kv_cache_dtype=kv,
                         device=torch.device("cuda:0"))


def _spec_run(torch, sr, target, draft, steps: int, warmup: int, kv: str, graphs: bool,
              max_model_len: int = 0) -> dict:
    """One timed config-3 run: prefill a 64-token prompt, two eager steps (they
    create every workspace), graph capture of the draft and verify phases, then
    `warmup` untimed and `steps` timed steps between HIP events on the stream."""
    gamma = 3
    dev = torch.device("cuda:0")
    max_len = 64 + (steps + warmup + 4) * (gamma + 1) + 8
    if max_model_len > 0 and max_len > max_model_len:
        raise ValueError(f"--steps/--warmup need {max_len} tokens, past --max-model-len")
    runner = _spec_runner(torch, sr, target, draft, kv, max_model_len, max_len)
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, 10000, (64,), generator=g).tolist()
    runner.load_prompts([prompt])
    runner.prefill()
    torch.manual_seed(0)
    for _ in range(2):  # eager steps create every workspace before capture
        runner.step()
    torch.cuda.synchronize()
    if graphs:
        runner.capture()
    run = runner.replay if graphs else runner.step
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    len0 = runner.lengths()[0]
    stream = torch.cuda.current_stream(dev)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(3 * steps)]
    e_start = torch.cuda.Event(enable_timing=True)
    e_end = torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    e_start.record(stream)
    for i in range(steps):
        evs[3 * i].record(stream)
        if graphs:
            runner.graphs[0].replay()
            evs[3 * i + 1].record(stream)
            runner.graphs[1].replay()
        else:
            runner.draft_phase()
            evs[3 * i + 1].record(stream)
            runner.verify_phase()
        evs[3 * i + 2].record(stream)
    e_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    runner.check()  # no acceptance call of the timed steps produced invalid outputs
    len1 = runner.lengths()[0]
    res = dict(graphs=graphs, gpu_ms=e_start.elapsed_time(e_end), len0=len0, len1=len1,
               emitted=len1 - len0, wall=wall,
               draft_ms=sum(evs[3 * i].elapsed_time(evs[3 * i + 1]) for i in range(steps)),
               verify_ms=sum(evs[3 * i + 1].elapsed_time(evs[3 * i + 2]) for i in range(steps)))
    del runner
    torch.cuda.empty_cache()
    return res


def _spec_full_run(torch, sr, target, draft, kv: str, max_model_len: int = 0,
                   output_tokens: int = 256, chunk: int = 16) -> dict:
    """Config 3 as stated: a 64-token prompt decoded to `output_tokens` completion
    tokens (max_tokens, so the sequence finishes exactly there as in
    llm_engine.py:154-160), every step through the HIP graphs after the two eager
    steps that precede capture. Each step is timed with HIP events on the stream and
    the context length after it is copied aside (outside the timed events); the GPU
    time of the steps up to the one that finished the sequence is the run's time."""
    gamma = 3
    dev = torch.device("cuda:0")
    runner = _spec_runner(torch, sr, target, draft, kv, max_model_len,
                          64 + output_tokens + gamma + 8)
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, 10000, (64,), generator=g).tolist()
    runner.load_prompts([prompt], max_tokens=output_tokens)
    runner.prefill()
    torch.manual_seed(0)
    eager_ms = []
    stream = torch.cuda.current_stream(dev)
    for _ in range(2):  # eager steps create every workspace before capture
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        runner.step()
        e1.record(stream)
        eager_ms.append((e0, e1))
    torch.cuda.synchronize()
    runner.capture()
    end = 64 + output_tokens
    lens, evs = [], []
    hist = torch.zeros(4 * output_tokens, dtype=torch.int32, device=dev)
    n = 0
    while True:
        for _ in range(chunk):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            runner.replay()
            e1.record(stream)
            hist[n:n + 1].copy_(runner.state.context_lens[:1])
            evs.append((e0, e1))
            n += 1
        torch.cuda.synchronize()
        lens = hist[:n].cpu().tolist()
        if lens[-1] >= end or n + chunk > hist.numel():
            break
    runner.check()
    if lens[-1] < end:
        raise RuntimeError(f"full run stopped at {lens[-1]} of {end} tokens")
    last = next(i for i, x in enumerate(lens) if x >= end)
    steps = 2 + last + 1
    gpu_ms = sum(a.elapsed_time(b) for a, b in eager_ms + evs[:last + 1])
    emitted = end - (64 + 1)  # the first completion token comes from the prefill
    res = dict(steps=steps, gpu_ms=gpu_ms, emitted=emitted,
               final_tokens=runner.lengths()[0])
    del runner
    torch.cuda.empty_cache()
    return res


def bench_spec(args, torch, hv):
    """Config 3: speculative decoding at batch 1 with random-init Qwen3-8B target and
    Qwen3-0.6B draft (or the forced-acceptance draft = target's first 28 layers)."""
    import importlib as _il
    q3 = _il.import_module("hilda-vllm_amd.engine.qwen3_host")
    sr = _il.import_module("hilda-vllm_amd.engine.spec_runner")
    dev = torch.device("cuda:0")
    gamma = 3
    t0 = time.perf_counter()
    target = q3.Qwen3Host(q3.QWEN3_8B, device=dev, seed=1)
    if args.draft == "forced":
        draft = q3.Qwen3Host(q3.QWEN3_8B, share_from=target, num_layers=args.draft_layers)
    else:
        draft = q3.Qwen3Host(q3.QWEN3_0_6B, device=dev, seed=2)
    torch.cuda.synchronize()
    init_s = time.perf_counter() - t0
    mml = args.max_model_len
    m = _spec_run(torch, sr, target, draft, args.steps, args.warmup, args.kv, not args.eager,
                  max_model_len=mml)
    graphs, gpu_ms, draft_ms, verify_ms = m["graphs"], m["gpu_ms"], m["draft_ms"], m["verify_ms"]
    len0, len1, emitted, wall = m["len0"], m["len1"], m["emitted"], m["wall"]
    tok_s = emitted / (gpu_ms / 1e3)
    accepted_drafts = emitted - args.steps
    full = None
    if not args.eager and not args.no_full_run:
        full = _spec_full_run(torch, sr, target, draft, args.kv, max_model_len=mml)
    # the step's in-scope kernels: the fused attention launch (one per layer) is the
    # headline roofline; acceptance and bookkeeping complete the in-scope step
    roof_attn_fused = attention_probe(torch, hv, kv=args.kv, fused=True)
    roof_attn = attention_probe(torch, hv, kv=args.kv)
    roof_inscope = inscope_step_probe(torch, hv, roof_attn_fused, target.g.num_layers)
    # the projections' weight stream (not part of the verify+accept object)
    roof_gemm = gemm_probe(torch, hv, target)
    step_bytes = target_step_bytes(target)
    step_us = verify_ms / args.steps * 1e3
    roof_step = {"bound": "hbm", "achieved": round(step_bytes / (step_us * 1e-6) / 1e9, 1),
                 "peak": HBM_PEAK_GBS, "unit": "GB/s",
                 "frac": round(step_bytes / (step_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                 "bytes_per_step": step_bytes, "step_us": round(step_us, 1),
                 "scope": "includes the projection and LM-head weights, which the "
                          "verify+accept object leaves out (see roofline_inscope_step)",
                 "what": "whole verify phase: the target's layer weights and LM head, each "
                         "read once per step, over the phase's HIP-event time"}
    res = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "accepted tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gpu_ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init N(0,0.02^2) weights, 64 uniform-random prompt ids)",
        "config": {"workload": "config 3: spec decode batch 1, Qwen3-8B target / "
                               f"{'Qwen3-0.6B' if args.draft != 'forced' else 'forced (target first 28 layers)'} draft",
                   "batch": 1, "gamma": gamma, "prompt_len": 64, "temperature": 0.6,
                   "acceptance": "reference", "kv_cache": args.kv,
                   "hip_graphs": graphs, "output_tokens_timed": emitted,
                   "context_range_timed": [len0, len1],
                   "max_model_len": mml if mml > 0 else "sized to the run",
                   "roofline_probe_context": PROBE_CONTEXT},
        "verify_accept_step_us": round(verify_ms / args.steps * 1e3, 1),
        # published reference numbers (RTX 5090, trained Qwen3-8B / 0.6B, 65.5% acceptance,
        # prompt 256): benchmarks/results/20260322T104708Z-spec-decode-batch1.json:40,45-49;
        # not the same hardware nor acceptance rate, hence vs_baseline stays null
        "reference_rtx5090": {"spec_decode_tok_s": 104.72, "verify_step_us": 17930.0,
                              "acceptance_rate": 0.655},
        "draft_step_us": round(draft_ms / args.steps * 1e3, 1),
        "tokens_emitted": emitted,
        "tokens_per_step": round(emitted / args.steps, 3),
        "acceptance_rate": round(accepted_drafts / (args.steps * gamma), 4),
        "context_len_end": len1,
        "wall_s": round(wall, 3),
        "init_s": round(init_s, 1),
        "roofline": roof_attn_fused,
        "roofline_inscope_step": roof_inscope,
        "roofline_attention_unfused": roof_attn,
        "roofline_gemm": roof_gemm,
        "roofline_step": roof_step,
    }
    if full is not None:
        res["full_run"] = {
            "what": "config 3 as stated: 64-token prompt to 256 completion tokens (the first "
                    "from the prefill), every spec step timed",
            "steps": full["steps"], "tokens_emitted": full["emitted"],
            "value": round(full["emitted"] / (full["gpu_ms"] / 1e3), 2),
            "unit": "accepted tok/s", "ms_per_step": round(full["gpu_ms"] / full["steps"], 4),
            "acceptance_rate": round((full["emitted"] - full["steps"]) / (full["steps"] * gamma),
                                     4),
            "final_context": full["final_tokens"]}
    if args.draft != "forced" and not args.no_forced:
        # config 3's second mode: the draft is the target's first 28 layers plus
        # its LM head, so most drafts are accepted and the accept path (bonus
        # tokens, long commits) runs every step; a shorter timed run
        fdraft = q3.Qwen3Host(q3.QWEN3_8B, share_from=target, num_layers=28)
        fs = min(args.steps, 64)
        f = _spec_run(torch, sr, target, fdraft, fs, 4, args.kv, not args.eager,
                      max_model_len=mml)
        res["forced_acceptance"] = {
            "draft": "target's first 28 layers + LM head", "steps": fs,
            "value": round(f["emitted"] / (f["gpu_ms"] / 1e3), 2), "unit": "accepted tok/s",
            "ms_per_step": round(f["gpu_ms"] / fs, 4),
            "verify_accept_step_us": round(f["verify_ms"] / fs * 1e3, 1),
            "draft_step_us": round(f["draft_ms"] / fs * 1e3, 1),
            "tokens_per_step": round(f["emitted"] / fs, 3),
            "acceptance_rate": round((f["emitted"] - fs) / (fs * gamma), 4)}
        del fdraft
    if not args.no_cpu_baseline:
        w = hv.synthetic.accept_workload(1, gamma, seed=0, dtype="bf16", temperature=0.6)
        res["cpu_baseline"] = cpu_baseline_accept(torch, w, args.cpu_seconds)
    return res


def bench_adaptive(args, torch, hv):
    """Config 4: adaptive-gamma batched speculative decoding, B sequences (default 32),
    prompts ~ U[32, 128], every sequence decoding to --max-context tokens (default
    8192) in an FP8-e4m3 target cache of 256-token blocks whose pool holds 3/4 of
    what all sequences need at the end (block pressure: sequences wait for blocks
    until others finish; when none can proceed the longest is preempted and later
    recomputed by prefill, scheduler.py:231-238,313-320). Random-init 8B target /
    0.6B draft (or, with --draft forced, the target's first 28 layers and LM head, so
    that drafts are accepted often enough for gamma to move up), T=0.6, reference
    acceptance, gamma from 3 adapted in [1, 7] (llm_engine.py:197-208 with the range
    of the config)."""
    import importlib as _il
    import numpy as np
    q3 = _il.import_module("hilda-vllm_amd.engine.qwen3_host")
    sr = _il.import_module("hilda-vllm_amd.engine.spec_runner")
    dev = torch.device("cuda:0")
    B, bs = args.batch if args.batch > 1 else 32, 256
    rng = np.random.default_rng(0)
    plens = rng.integers(32, 129, size=B)
    prompts = [rng.integers(0, 10000, size=n).tolist() for n in plens]
    ctx = args.max_context
    need = sum(-(-(ctx + 9) // bs) for _ in range(B))
    num_blocks = max(int(0.75 * need), sum(-(-int(n) // bs) for n in plens) + B)
    target = q3.Qwen3Host(q3.QWEN3_8B, device=dev, seed=1)
    if args.draft == "forced":
        draft = q3.Qwen3Host(q3.QWEN3_8B, share_from=target, num_layers=args.draft_layers)
    else:
        draft = q3.Qwen3Host(q3.QWEN3_0_6B, device=dev, seed=2)
    runner = sr.SpecRunner(target, draft, batch=B, gamma=3, max_model_len=ctx + 16, block_size=bs,
                           kv_cache_dtype="fp8", num_blocks=num_blocks, temperature=0.6,
                           mode="reference", adaptive=True, max_gamma=7, device=dev)
    runner.load_prompts(prompts)
    runner.state.max_tokens.copy_(torch.tensor([ctx - int(n) for n in plens], dtype=torch.int32))
    runner.prefill()
    len0 = sum(runner.lengths())
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    waited = preemptions = readmitted = 0
    t0 = time.perf_counter()
    e0.record(stream)
    steps = 0
    while steps < args.steps:
        if runner.preempted:
            readmitted += runner.readmit()
        if bool(runner.state.finished.all()) and not runner.preempted:
            break
        runner.step_graph()
        G = runner._per_gamma[runner.history[-1][0]]
        fin = runner.state.finished
        waited += int(((G.elig == 0) & (fin == 0)).sum())
        if int(G.elig.sum()) == 0 and not bool(fin.all()):
            # no sequence could get its blocks: preempt the longest (scheduler.py:231-238
            # preempts at the first miss; here sequences wait until none can proceed)
            lens = runner.state.context_lens.masked_fill(fin.bool(), -1)
            runner.preempt(int(torch.argmax(lens)))
            preemptions += 1
        steps += 1
        if steps % 200 == 0:
            print(f"[adaptive] step {steps} tokens {sum(runner.lengths()) - len0} "
                  f"gamma {runner.gamma} preempted {preemptions} readmitted {readmitted}",
                  file=sys.stderr, flush=True)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = e0.elapsed_time(e1)
    emitted = sum(runner.lengths()) - len0
    gam = [h[0] for h in runner.history]
    acc = sum(h[1] for h in runner.history)
    prop = sum(h[2] for h in runner.history)
    return {"metric": "adaptive-gamma batched spec decode tokens/s (config 4)",
            "value": round(emitted / (gpu_ms / 1e3), 2), "unit": "tok/s (all sequences)",
            "n_gpus": 1, "steps": steps, "warmup": 0, "ms_per_step": round(gpu_ms / max(steps, 1), 3),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16, fp8-e4m3 KV",
            "data": "synthetic (random-init weights, uniform-random prompt ids)",
            "config": {"workload": "config 4: adaptive gamma, FP8 KV, block pressure", "batch": B,
                       "max_context": ctx, "num_blocks": num_blocks, "blocks_needed_at_end": need,
                       "draft": f"target's first {args.draft_layers} layers + LM head"
                       if args.draft == "forced" else "Qwen3-0.6B"},
            "tokens_emitted": emitted,
            "all_finished": bool(runner.state.finished.all()) and not runner.preempted,
            "preemptions": preemptions, "readmissions": readmitted,
            "gamma_histogram": {str(k): gam.count(k) for k in sorted(set(gam))},
            "acceptance_rate": round(acc / max(prop, 1), 4), "sequence_steps_waiting_for_blocks": waited,
            "wall_s": round(wall, 2)}


PROBE_CONTEXT = 320  # config-3 end state: 64 prompt tokens + 256 generated tokens


def target_step_bytes(target) -> int:
    """Bytes a verify step of the target must read at least once: every layer's
    projection weights and the LM head (bf16)."""
    n = target.lm_head.numel()
    for lyr in target.layers:
        n += lyr.qkv.numel() + lyr.o.numel() + lyr.gate_up.numel() + lyr.down.numel()
    return 2 * n


class _GateUpLayer:
    """One layer's gate/up weight and post-attention norm weight."""

    def __init__(self, gate_up, ln2):
        self.gate_up = gate_up
        self.ln2 = ln2


class _GateUpLayers:
    """The gate/up weights (and post-attention norm weights) of an 8B-shaped target,
    N(0, 0.02^2) bf16, without the rest of the model (the gemm workload)."""

    def __init__(self, torch, g, device):
        gen = torch.Generator(device=device).manual_seed(4)
        self.g = g
        self.layers = [
            _GateUpLayer((torch.randn((2 * g.ffn, g.hidden), generator=gen, device=device)
                          * 0.02).to(torch.bfloat16),
                         torch.ones(g.hidden, dtype=torch.bfloat16, device=device))
            for _ in range(g.num_layers)]


def bench_gemm(args, torch, hv):
    """The spec step's dominant kernel alone (gemm_probe over 36 fresh weight sets)."""
    q3 = importlib.import_module("hilda-vllm_amd.engine.qwen3_host")
    model = _GateUpLayers(torch, q3.QWEN3_8B, torch.device("cuda:0"))
    roof = gemm_probe(torch, hv, model, reps=max(1, args.steps // 36))
    return {"metric": METRIC, "value": roof["avg_launch_us"],
            "unit": "us/launch (gate/up projection)", "n_gpus": 1, "steps": roof["launches"],
            "warmup": 36, "ms_per_step": roof["avg_launch_us"] / 1e3, "higher_is_better": False,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (N(0,0.02^2) weights, N(0,1) rows)",
            "config": {"workload": "gate/up projection of the 8B target at the verify shape, "
                                   "36 layers"},
            "roofline": roof}


def gemm_probe(torch, hv, target, rows: int = 4, reps: int = 10):
    """The step's dominant kernel (the largest share of the step's kernel time,
    profiles/trace_spec-config3.md): the target's gate/up projection at the verify
    shape (4 rows, K = 4096, 2 x 12288 weight rows, RMSNorm with the residual add in
    its prologue, SwiGLU in its epilogue). One launch per layer over the target's own
    36 weight matrices (as in one verify step), captured in a HIP graph and replayed
    `reps` times between two HIP events on the launch stream."""
    dev = torch.device("cuda:0")
    g = target.g
    gen = torch.Generator(device=dev).manual_seed(3)
    h = torch.randn((rows, g.hidden), generator=gen, device=dev).to(torch.bfloat16)
    res = torch.randn((rows, g.hidden), generator=gen, device=dev).to(torch.bfloat16)
    layers = list(target.layers)

    def launch_all():
        for lyr in layers:
            hv.ops.linear_rmsnorm(h, lyr.ln2, g.rms_eps, lyr.gate_up, residual=res, swiglu=True)

    us = graph_time_us(torch, dev, launch_all, reps) / len(layers)
    # weights, norm weight, input and residual rows in, residual rows and SwiGLU rows out
    per_launch = 2 * (2 * g.ffn * g.hidden + g.hidden + 3 * rows * g.hidden + rows * g.ffn)
    achieved = per_launch / (us * 1e-6) / 1e9
    kernel = "k_skinny<4, 1, 1, true, true>"
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": profiled_traffic(kernel, "gemm-gate-up"),
            "kernel": kernel, "bytes_per_launch": per_launch, "avg_launch_us": round(us, 3),
            "shape": f"M={rows} K={g.hidden} N=2x{g.ffn} (gate/up, RMSNorm prologue, SwiGLU)",
            "launches": reps * len(layers)}


def attention_probe(torch, hv, kv: str = "auto", L: int = PROBE_CONTEXT, layers: int = 36,
                    reps: int = 20, fused: bool = False):
    """The verify-attention kernel at the batch-1 verify shape of the 8B target
    (B=1, gamma+1=4 queries, 32 Q / 8 KV heads, D=128, context L, 256-token blocks):
    one launch per layer over `layers` separate random caches (as in one verify
    step), captured in a HIP graph and replayed `reps` times between two HIP events
    on the launch stream. avg_launch_us includes the graph's per-node dispatch gap.
    fused: the launch the spec step runs, hs_qk_norm_rope_attend (q/k-norm + RoPE
    of the 4 qkv rows, their k/v stored at keys L-4 .. L-1, then the attention);
    its bytes add the qkv rows read and the k/v rows stored, less the q read."""
    dev = torch.device("cuda:0")
    R, Hq, Hkv, D, bs = 4, 32, 8, 128, 256
    nb = (L + bs - 1) // bs
    gen = torch.Generator(device=dev).manual_seed(1)
    fp8 = kv == "fp8"
    caches = []
    for _ in range(layers):
        k = torch.randn((nb, bs, Hkv, D), generator=gen, device=dev)
        v = torch.randn((nb, bs, Hkv, D), generator=gen, device=dev)
        dt = torch.float8_e4m3fn if fp8 else torch.bfloat16
        caches.append((k.to(dt), v.to(dt)))
    q = torch.randn((R, Hq, D), generator=gen, device=dev).to(torch.bfloat16)
    cu_q = torch.tensor([0, R], dtype=torch.int32, device=dev)
    cu_k = torch.tensor([0, L], dtype=torch.int32, device=dev)
    bt = torch.randperm(nb, generator=torch.Generator().manual_seed(2)).to(torch.int32)
    bt = bt.view(1, nb).to(dev)
    outs = [torch.empty((R, Hq, D), dtype=torch.bfloat16, device=dev) for _ in range(layers)]

    skv = 1 if fp8 else 2
    if fused:
        qkv = torch.randn((R, (Hq + 2 * Hkv) * D), generator=gen, device=dev).to(torch.bfloat16)
        qw = torch.ones(D, dtype=torch.bfloat16, device=dev)
        inv = 1.0 / (1e6 ** (torch.arange(0, D, 2, dtype=torch.float32, device=dev) / D))
        f = torch.outer(torch.arange(L, dtype=torch.float32, device=dev), inv)
        cs = torch.cat([f.cos(), f.sin()], -1).contiguous()
        pos = torch.arange(L - R, L, dtype=torch.int64, device=dev)
        btc = bt.view(-1).cpu()
        slots = torch.tensor([int(btc[p // bs]) * bs + p % bs for p in range(L - R, L)],
                             dtype=torch.int32, device=dev)

        def launch_all():
            for i, (k, v) in enumerate(caches):
                hv.ops.qk_norm_rope_attend(qkv, Hq, Hkv, qw, qw, cs, pos, 1e-6, k, v, slots, bt,
                                           cu_q, cu_k, R, L, D ** -0.5, out=outs[i])
        per_launch = (L * Hkv * D * 2 * skv + R * (Hq + 2 * Hkv) * D * 2 + R * Hq * D * 2
                      + R * 2 * Hkv * D * skv)
        kernel = f"k_verify_attn_qkv<{'true' if fp8 else 'false'}, 4>"
    else:
        def launch_all():
            for i, (k, v) in enumerate(caches):
                hv.ops.verify_attention(q, k, v, bt, cu_q, cu_k, R, L, D ** -0.5, out=outs[i])
        per_launch = L * Hkv * D * 2 * skv + 2 * R * Hq * D * 2
        kernel = f"k_verify_attn<{'true' if fp8 else 'false'}, 4>"

    us = graph_time_us(torch, dev, launch_all, reps) / layers
    achieved = per_launch / (us * 1e-6) / 1e9
    workload = "attention-b1-fused" if fused else "attention-b1"
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 5), "traffic": profiled_traffic(kernel, workload),
            "mfma_util": profiled_counter(kernel, workload, "MfmaUtil %"),
            "kernel": kernel, "bytes_per_launch": per_launch, "avg_launch_us": round(us, 3),
            "shape": f"B=1 q={R} Hq={Hq} Hkv={Hkv} D={D} L={L} block {bs}",
            "launches": reps * layers}


def _accept_args(**kw):
    """Arguments of the acceptance workload (bench_accept) at the spec step's shape."""
    ns = argparse.Namespace(batch=1, gamma=3, mode="reference", logits="bf16", per_seq=False,
                            temperature=0.6, top_k=0, top_p=1.0, chain=False,
                            no_topk_hint=False, no_cpu_baseline=True, steps=200, warmup=20,
                            cpu_seconds=0.0)
    for k, v in kw.items():
        setattr(ns, k, v)
    return ns


def _probe_state(torch, hv, dev, context: int, end: int):
    """A batch-1 sequence of `context` tokens (random ids, never finishing) in a
    256-token-block state with blocks for `end` tokens free behind it."""
    bs = 256
    W = (end + bs - 1) // bs + 1
    st = hv.ops.SpecStateTensors(1, W, end + 8, W + 2, bs, -1, dev)
    nblk = (context + bs - 1) // bs
    bt = torch.full((1, W), -1, dtype=torch.int32)
    bt[0, :nblk] = torch.arange(nblk, dtype=torch.int32)
    st.block_tables.copy_(bt)
    st.num_seq_blocks.fill_(nblk)
    st.context_lens.fill_(context)
    st.num_prompt.fill_(64)
    st.max_tokens.fill_(1 << 30)
    st.ignore_eos.fill_(1)
    st.tokens.copy_(torch.randint(0, V, st.tokens.shape, generator=torch.Generator().manual_seed(5)))
    ring = torch.zeros(W + 2, dtype=torch.int32)
    ring[:W + 2 - nblk] = torch.arange(nblk, W + 2, dtype=torch.int32)
    st.free_ring.copy_(ring)
    st.free_hdr.copy_(torch.tensor([0, W + 2 - nblk], dtype=torch.int32))
    ref = torch.zeros(W + 2, dtype=torch.int32)
    ref[:nblk] = 1
    st.ref_count.copy_(ref)
    return st


def _probe_stages(torch, dev, gamma: int):
    """Staging buffers of the next draft step (look-back: two rows) and the next
    verify step (gamma + 1 rows) at batch 1."""
    R = gamma + 1
    i64 = dict(dtype=torch.int64, device=dev)
    i32 = dict(dtype=torch.int32, device=dev)
    stage0 = (torch.empty(2, **i64), torch.empty(2, **i64), torch.empty(2, **i32),
              torch.empty(2, **i32), torch.empty(2, **i32))
    vstage = (torch.empty(R, **i64), torch.empty(R, **i64), torch.empty(R, **i32),
              torch.empty(2, **i32), torch.empty(2, **i32))
    return stage0, vstage


def _bookkeeping_bytes(W: int, gamma: int, out_len: int) -> int:
    """State words, staging rows and committed tokens one batch-1 step's bookkeeping
    reads and writes."""
    R = gamma + 1
    return (4 * 6 + 4 * W  # prealloc: lengths, counts, free header, table row, ref counts
            + 8 + R * (8 + 4) + 8 + 2 * 2 * 4  # verify staging: last id, positions, slots, cu
            + R * 8 + 4 + out_len * 8 + 4 * 6  # commit: emitted tokens in, tokens appended
            + 2 * (8 + 8 + 4) + 2 * 2 * 4)  # next draft step 0: ids, positions, slots, cu


def bookkeeping_probe(torch, hv, context: int = PROBE_CONTEXT - 4, gamma: int = 3,
                      out_len: int = 2, reps: int = 20):
    """The spec step's bookkeeping at batch 1 as its own launch: one
    hs_spec_commit_next after the acceptance (the commit, then the next step's
    pre-allocation, first draft-step staging and verify staging; the draft steps
    write the draft tokens' ids in place), as the fixed-gamma runner makes it when
    the acceptance cannot take it (batch above 1), graph-timed from a sequence of
    `context` tokens; every step commits `out_len` tokens (one accepted draft and the
    resample, the typical outcome). One graph holds `per_graph` steps, so a replay
    keeps the GPU busy longer than the host takes to launch the next one. Returns
    (µs per step, bytes per step)."""
    dev = torch.device("cuda:0")
    per_graph = 32
    end = context + (reps + 3) * per_graph * out_len + gamma + 2
    st = _probe_state(torch, hv, dev, context, end)
    elig = torch.empty(1, dtype=torch.int32, device=dev)
    draft = torch.randint(0, V, (1, gamma), dtype=torch.int64, device=dev)
    out = torch.randint(0, V, (1, gamma + 1), dtype=torch.int64, device=dev)
    olen = torch.full((1,), out_len, dtype=torch.int32, device=dev)
    stage0, vstage = _probe_stages(torch, dev, gamma)
    hv.ops.spec_prealloc(st, gamma, out=elig)  # the step before the first replay
    vstage[0][1:].copy_(draft[0])  # the draft steps' in-place ids

    def steps():
        for _ in range(per_graph):
            hv.ops.spec_commit_next(st, gamma, out, olen, elig, gamma, stage0, lookback=True,
                                    stage_verify=vstage)

    us = graph_time_us(torch, dev, steps, reps) / per_graph
    return us, _bookkeeping_bytes(st.W, gamma, out_len)


def accept_commit_probe(torch, hv, reps: int = 2):
    """The batch-1 step's acceptance with its bookkeeping, as the fixed-gamma runner
    makes it: one hs_spec_accept_commit_next per step, a single launch (the
    workgroup that writes the acceptance outputs commits them, pre-allocates and
    stages the next step). Inputs are rotated as in bench_accept so that every call
    reads its rows from HBM; the sequence starts at PROBE_CONTEXT - 4 tokens and
    grows by the tokens each call emits. Returns (µs per step, bytes per step: the
    acceptance's rows and the bookkeeping's words, the latter at the typical two
    emitted tokens, accepted mean)."""
    dev = torch.device("cuda:0")
    args = _accept_args()
    g = args.gamma
    R = g + 1
    step_bytes = R * V * 2 + g * V * 4
    copies = max(2, int(512e6 // step_bytes) + 1)
    target, q, s = _accept_inputs(torch, hv, dev, args)
    bufs = [(target.clone(), q.clone()) for _ in range(copies)]
    del target, q
    context = PROBE_CONTEXT - 4
    end = context + copies * (reps + 3) * R + R + 2
    st = _probe_state(torch, hv, dev, context, end)
    elig = torch.empty(1, dtype=torch.int32, device=dev)
    stage0, vstage = _probe_stages(torch, dev, g)
    hv.ops.spec_prealloc(st, g, out=elig)
    cn = dict(state=st, eligible=elig, next_gamma=g, stage0=stage0, lookback=True,
              stage_verify=vstage)
    outs = []

    def one_round():
        outs.clear()
        for i in range(copies):
            lg, qq = bufs[i]
            outs.append(hv.ops.spec_accept(lg, qq, s["draft_tokens"], s["temperatures"],
                                           s["u_accept"], s["u_resample"], commit_next=cn))

    us = graph_time_us(torch, dev, one_round, reps) / copies
    hv.ops.check_accepted(outs[-1][0], "accept_commit_probe")
    emitted = float(sum(int(o[2][0]) for o in outs)) / len(outs)
    return us, step_bytes + _bookkeeping_bytes(st.W, g, 2), round(emitted, 3)


def inscope_step_probe(torch, hv, attn_roof: dict, layers: int):
    """The verify+accept step's own work at batch 1, gamma 3, context PROBE_CONTEXT:
    `layers` fused attention launches (q/k-norm + RoPE + KV store + attention, each
    `attn_roof`'s bytes and graph-timed average), then the acceptance (bf16 target
    rows and f32 draft rows, (gamma+1)V*2 + gamma*V*4 bytes; inputs rotated so every
    call reads HBM) with the step's bookkeeping in the same launch
    (accept_commit_probe). The projection and LM-head weights are left out. achieved
    = in-scope bytes over the sum of those kernels' graph-timed durations (each
    including its graph node's dispatch gap, as in the step). The acceptance and the
    bookkeeping as separate launches are reported beside it."""
    acc = bench_accept(_accept_args(), torch, hv)
    acc_us = acc["value"]
    acc_bytes = acc["roofline"]["bytes_per_step"]
    bk_us, bk_bytes = bookkeeping_probe(torch, hv)
    ac_us, ac_bytes, emitted = accept_commit_probe(torch, hv)
    attn_us = layers * attn_roof["avg_launch_us"]
    attn_bytes = layers * attn_roof["bytes_per_launch"]
    nbytes = attn_bytes + ac_bytes
    us = attn_us + ac_us
    achieved = nbytes / (us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 5), "bytes_per_step": nbytes,
            "us_per_step": round(us, 2),
            "parts": {"attention": {"launches": layers, "bytes": attn_bytes,
                                    "us": round(attn_us, 2)},
                      "acceptance_and_bookkeeping": {"launches": 1, "bytes": ac_bytes,
                                                     "us": round(ac_us, 2),
                                                     "emitted_mean": emitted},
                      "as_two_launches": {"acceptance_us": round(acc_us, 2),
                                          "acceptance_bytes": acc_bytes,
                                          "bookkeeping_us": round(bk_us, 2),
                                          "bookkeeping_bytes": bk_bytes}},
            "what": f"verify+accept step without the projection weights: {layers} fused "
                    f"attention launches at L={PROBE_CONTEXT}, then the acceptance with the "
                    "commit, the next step's pre-allocation, draft staging and verify staging "
                    "in one launch; graph-timed per part (as_two_launches: the acceptance and "
                    "the bookkeeping timed as separate launches, not summed)"}


def profiled_traffic(kernel: str, workload: str):
    """HBM bytes per launch of `kernel` in `workload` from the committed rocprofv3
    counter summary profiles/traffic.md (FETCH_SIZE and WRITE_SIZE in KiB per
    dispatch, each scaled by the factor a plain 256 MiB copy gives), or None."""
    path = ROOT / "profiles" / "traffic.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 5 and cells[0] == workload and cells[1] == kernel:
            try:
                return int(float(cells[4]))
            except ValueError:
                return None
    return None


def profiled_counter(kernel: str, workload: str, column: str):
    """A compute counter (column "MfmaUtil %" or "VALUBusy %") of `kernel` in
    `workload` from the compute-counter table of profiles/traffic.md, or None."""
    path = ROOT / "profiles" / "traffic.md"
    if not path.exists():
        return None
    header = None
    for line in path.read_text().splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 3 and cells[:2] == ["workload", "kernel"]:
            header = cells
            continue
        if header and column in header and len(cells) == len(header) and \
                cells[0] == workload and cells[1] == kernel:
            try:
                return float(cells[header.index(column)])
            except ValueError:
                return None
    return None


def call_traffic(kernels, workload: str):
    """HBM bytes of one call made of `kernels` (the sum of their profiled rows), or None."""
    rows = [profiled_traffic(k, workload) for k in kernels]
    return None if any(r is None for r in rows) else sum(rows)


def bench_attention_b1(args, torch, hv):
    roof = attention_probe(torch, hv, kv=args.kv, reps=max(1, args.steps // 36),
                           fused=args.attn_fused)
    return {"metric": METRIC, "value": roof["avg_launch_us"], "unit": "us/launch (verify attention)",
            "n_gpus": 1, "steps": roof["launches"], "warmup": 36, "ms_per_step": roof["avg_launch_us"] / 1e3,
            "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
            "dtype": "fp8-e4m3 KV, bf16 MFMA" if args.kv == "fp8" else "bf16",
            "data": "synthetic (seeded N(0,1) q/k/v, random block permutation)",
            "config": {"workload": "verify attention at the config-3 batch-1 verify shape, 36 layers"
                       + (" (q/k-norm + RoPE + KV store in the prologue)" if args.attn_fused else ""),
                       "kv_cache": args.kv, "context": PROBE_CONTEXT},
            "roofline": roof}


def bench_copy(args, torch, hv):
    """Plain device-to-device copy of 256 MiB (the calibration kernel for the HBM
    byte counters): GB/s counts the bytes read plus the bytes written."""
    dev = torch.device("cuda:0")
    n = 256 << 20
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    us = graph_time_us(torch, dev, lambda: dst.copy_(src), max(1, args.steps))
    gbs = 2 * n / (us * 1e-6) / 1e9
    return {"metric": "device copy bandwidth (calibration)", "value": round(gbs, 1), "unit": "GB/s",
            "n_gpus": 1, "steps": max(1, args.steps), "warmup": 1, "ms_per_step": round(us / 1e3, 4),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u8",
            "data": "synthetic", "config": {"workload": "copy 256 MiB", "bytes_read": n,
                                            "bytes_written": n}}


def _csv_rows(path):
    import csv
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def rocprof_summary(directory: str, kernel_filter: str | None = None) -> str:
    """Text summary of a rocprofv3 CSV output directory (--output-format csv):
    per-kernel dispatch statistics (kernel_stats.csv), per-grid statistics of the
    kernels matching `kernel_filter` (kernel_trace.csv) and per-kernel averages
    of collected counters (counter_collection.csv)."""
    import glob
    out = []
    stats = sorted(glob.glob(os.path.join(directory, "**", "*kernel_stats.csv"), recursive=True))
    if stats:
        rows = _csv_rows(stats[0])
        total = sum(float(r["TotalDurationNs"]) for r in rows)
        out.append(f"kernel dispatch statistics ({os.path.basename(stats[0])}), "
                   f"total {total / 1e3:.1f} us")
        out.append(f"{'calls':>7} {'avg_us':>9} {'min_us':>9} {'max_us':>9} {'share':>6}  kernel")
        for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"]))[:25]:
            out.append(f"{int(r['Calls']):>7} {float(r['AverageNs']) / 1e3:>9.2f} "
                       f"{float(r['MinNs']) / 1e3:>9.2f} {float(r['MaxNs']) / 1e3:>9.2f} "
                       f"{100 * float(r['TotalDurationNs']) / total:>5.1f}%  {r['Name'][:110]}")
    trace = sorted(glob.glob(os.path.join(directory, "**", "*kernel_trace.csv"), recursive=True))
    if trace and kernel_filter:
        groups = {}
        for r in _csv_rows(trace[0]):
            if kernel_filter not in r["Kernel_Name"]:
                continue
            key = (r["Kernel_Name"][:80], r["Grid_Size_X"], r["Grid_Size_Y"], r["Grid_Size_Z"])
            groups.setdefault(key, []).append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
        out.append("")
        out.append(f"per-grid statistics of kernels matching '{kernel_filter}' (grid in work-items)")
        for (name, gx, gy, gz), d in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
            out.append(f"{len(d):>7} {sum(d) / len(d) / 1e3:>9.2f} {min(d) / 1e3:>9.2f} "
                       f"{max(d) / 1e3:>9.2f}  grid=({gx},{gy},{gz}) {name}")
    cc = sorted(glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True))
    if cc:
        agg = {}
        for r in _csv_rows(cc[0]):
            if kernel_filter and kernel_filter not in r["Kernel_Name"]:
                continue
            key = (r["Kernel_Name"][:100], r["Counter_Name"])
            agg.setdefault(key, []).append(float(r["Counter_Value"]))
        out.append("")
        out.append("counter averages per dispatch")
        out.append(f"{'dispatches':>10} {'average':>14} {'min':>14} {'max':>14}  counter  kernel")
        for (name, cname), v in sorted(agg.items(), key=lambda kv: -sum(kv[1]))[:25]:
            out.append(f"{len(v):>10} {sum(v) / len(v):>14.2f} {min(v):>14.2f} {max(v):>14.2f}  "
                       f"{cname}  {name}")
    return "\n".join(out)


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default="spec",
                    choices=["spec", "accept", "sampler", "attention", "attention-b1", "gemm",
                             "copy", "adaptive"])
    ap.add_argument("--max-context", type=int, default=8192)
    ap.add_argument("--rocprof-summary", metavar="DIR", default=None,
                    help="print a text summary of a rocprofv3 CSV output directory and exit")
    ap.add_argument("--kernel", default=None, help="kernel-name filter for --rocprof-summary")
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--gamma", type=int, default=3)
    ap.add_argument("--mode", default="reference", choices=["reference", "filtered", "greedy"])
    ap.add_argument("--logits", default="bf16", choices=["bf16", "f32"])
    ap.add_argument("--per-seq", action="store_true")
    ap.add_argument("--temperature", type=float, default=0.6)
    ap.add_argument("--top-k", type=int, default=0)
    ap.add_argument("--top-p", type=float, default=1.0)
    ap.add_argument("--draft", default="qwen3-0.6b", choices=["qwen3-0.6b", "forced"])
    ap.add_argument("--draft-layers", type=int, default=28,
                    help="--draft forced: the target's first N layers (36: the target itself)")
    ap.add_argument("--kv", default="auto", choices=["auto", "fp8"])
    ap.add_argument("--attn-fused", action="store_true",
                    help="attention-b1: the fused launch (hs_qk_norm_rope_attend) of the spec step")
    ap.add_argument("--eager", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--max-model-len", type=int, default=4096,
                    help="spec/adaptive: the runner's max_model_len (block tables, attention "
                         "launch plans); the reference's benchmarks use 4096; 0 = sized to the run")
    ap.add_argument("--no-full-run", action="store_true",
                    help="spec: skip the 256-token full-run companion")
    ap.add_argument("--no-forced", action="store_true",
                    help="spec workload: skip the forced-acceptance companion run")
    ap.add_argument("--chain", action="store_true",
                    help="accept and sampler workloads: force the launch chain (no single-launch kernel)")
    ap.add_argument("--no-topk-hint", action="store_true",
                    help="accept workload: do not pass the top-k <= 64 promise (chain path)")
    args = ap.parse_args(argv)
    if args.rocprof_summary:
        print(rocprof_summary(args.rocprof_summary, args.kernel))
        return 0
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; the verify path shards "
                          "by sequence / KV head across GPUs by design but no multi-GPU run "
                          "is part of it", "n_gpus": args.gpus}))
        return 2
    if args.steps is None:
        # spec: ~256 generated tokens over warm-up + timed steps at random-weight acceptance
        args.steps = {"spec": 180, "attention-b1": 720, "gemm": 360,
                      "adaptive": 1 << 30}.get(args.workload, 200)
    if args.warmup is None:
        args.warmup = 8 if args.workload == "spec" else 20
    import torch
    hv = importlib.import_module("hilda-vllm_amd")
    if args.workload == "spec":
        res = bench_spec(args, torch, hv)
    elif args.workload == "attention":
        res = bench_attention(args, torch, hv)
    elif args.workload == "copy":
        res = bench_copy(args, torch, hv)
    elif args.workload == "attention-b1":
        res = bench_attention_b1(args, torch, hv)
    elif args.workload == "gemm":
        res = bench_gemm(args, torch, hv)
    elif args.workload == "adaptive":
        res = bench_adaptive(args, torch, hv)
    elif args.workload == "sampler":
        res = bench_sampler(args, torch, hv)
    else:
        res = bench_accept(args, torch, hv)
    print(json.dumps(res))
    return 0


if __name__ == "__main__":
    sys.exit(main())
