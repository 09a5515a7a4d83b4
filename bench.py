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
  attention - config 2: paged verify attention, B=64, 4 queries, 16 Q / 8 KV
            heads, D=128, context ~ U[64, 2048], 256-token blocks in a random
            permutation, bf16 or (--kv fp8) fp8-e4m3 cache.
Timed launches are captured in HIP graphs and replayed between two HIP events
on the launch stream; inputs rotate over enough copies that every step reads
HBM (the MI355X MALL is 256 MB).
The roofline figure is algorithmic bytes per step divided by the HIP-event
time of the step measured on the launch stream; cpu_baseline times the
torch-CPU restatement of the reference loop (oracle/torch_port.py) on the
host cores of the same machine on a bounded sample.
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

    def step(i):
        lg, qq = bufs[i % copies]
        return hv.ops.spec_accept(lg, qq, s["draft_tokens"], s["temperatures"], s["u_accept"],
                                  s["u_resample"], mode=args.mode, top_ks=s["top_ks"],
                                  top_ps=s["top_ps"])

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
                   "input_copies_rotated": copies},
        "accepted_mean": round(sum(nacc) / len(nacc), 3),
        "wall_s": round(wall, 3),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": None, "bytes_per_step": step_bytes,
                     "kernels": "one hs_spec_accept call (row statistics, filter when "
                                "filtered, decision + resample partials, final search)"},
    }
    if not args.no_cpu_baseline:
        w = hv.synthetic.accept_workload(1, 3, seed=0, dtype="bf16", temperature=0.6)
        res["cpu_baseline"] = cpu_baseline_accept(torch, w, args.cpu_seconds)
    return res


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
    return {
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
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "bytes_per_launch": per_launch,
                     "kernel": f"k_verify_attn<{'true' if fp8 else 'false'}, 2> (+ k_attn_combine when split)"},
    }


def cpu_baseline_accept(torch, w, seconds: float):
    from oracle import torch_port
    cores = os.cpu_count() or 1
    cores = min(cores, 16)
    torch.set_num_threads(cores)
    lg = torch.from_numpy(w["logits"])  # bf16-rounded values as f32
    lg = lg.to(torch.bfloat16)
    q = torch.from_numpy(w["draft_probs"])
    dt = torch.from_numpy(w["draft_tokens"])
    T = torch.from_numpy(w["temperatures"])
    ua = torch.from_numpy(w["u_accept"])
    ur = torch.from_numpy(w["u_resample"])
    for _ in range(3):
        torch_port.run_verify_accept(lg, q, dt, T, ua, ur)
    n = 0
    t0 = time.perf_counter()
    while True:
        torch_port.run_verify_accept(lg, q, dt, T, ua, ur)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds and n >= 5:
            break
    return {"value": round(el / n * 1e6, 1), "unit": "us/step (fused acceptance)",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{n} acceptance steps at B=1 gamma=3 V=151936 over {el:.1f} s "
                      "(torch-CPU restatement of model_runner.py:391-428)"}


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
        draft = q3.Qwen3Host(q3.QWEN3_8B, share_from=target, num_layers=28)
    else:
        draft = q3.Qwen3Host(q3.QWEN3_0_6B, device=dev, seed=2)
    torch.cuda.synchronize()
    init_s = time.perf_counter() - t0
    max_len = 64 + (args.steps + args.warmup + 4) * (gamma + 1) + 8
    runner = sr.SpecRunner(target, draft, batch=1, gamma=gamma, max_model_len=max_len,
                           temperature=0.6, mode="reference", kv_cache_dtype=args.kv,
                           device=dev)
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, 10000, (64,), generator=g).tolist()
    runner.load_prompts([prompt])
    runner.prefill()
    torch.manual_seed(0)
    for _ in range(2):  # eager steps create every workspace before capture
        runner.step()
    torch.cuda.synchronize()
    graphs = not args.eager
    if graphs:
        runner.capture()
    run = runner.replay if graphs else runner.step
    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    len0 = runner.lengths()[0]
    stream = torch.cuda.current_stream(dev)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(3 * args.steps)]
    e_start = torch.cuda.Event(enable_timing=True)
    e_end = torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    e_start.record(stream)
    for i in range(args.steps):
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
    gpu_ms = e_start.elapsed_time(e_end)
    len1 = runner.lengths()[0]
    emitted = len1 - len0
    draft_ms = sum(evs[3 * i].elapsed_time(evs[3 * i + 1]) for i in range(args.steps))
    verify_ms = sum(evs[3 * i + 1].elapsed_time(evs[3 * i + 2]) for i in range(args.steps))
    tok_s = emitted / (gpu_ms / 1e3)
    accepted_drafts = emitted - args.steps
    roof = attention_probe(torch, hv, runner, len1)
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
                   "hip_graphs": graphs},
        "verify_accept_step_us": round(verify_ms / args.steps * 1e3, 1),
        "draft_step_us": round(draft_ms / args.steps * 1e3, 1),
        "tokens_emitted": emitted,
        "tokens_per_step": round(emitted / args.steps, 3),
        "acceptance_rate": round(accepted_drafts / (args.steps * gamma), 4),
        "context_len_end": len1,
        "wall_s": round(wall, 3),
        "init_s": round(init_s, 1),
        "roofline": roof,
    }
    if not args.no_cpu_baseline:
        w = hv.synthetic.accept_workload(1, gamma, seed=0, dtype="bf16", temperature=0.6)
        res["cpu_baseline"] = cpu_baseline_accept(torch, w, args.cpu_seconds)
    return res


def attention_probe(torch, hv, runner, L):
    """Average duration of the verify-attention kernel at the verify shape of this run
    (B=1, gamma+1=4 queries, 32 Q / 8 KV heads, context L) over the target's 36 layer
    caches: 36 launches captured in a HIP graph, replayed 20 times between two HIP
    events on the launch stream (per-launch time includes the graph's launch gaps)."""
    dev = runner.device
    g = runner.target.g
    R = runner.gamma + 1
    reps = 20
    q = torch.randn((R, g.num_heads, g.head_dim), device=dev).to(torch.bfloat16)
    cu_q = torch.tensor([0, R], dtype=torch.int32, device=dev)
    cu_k = torch.tensor([0, L], dtype=torch.int32, device=dev)
    bt = runner.state.block_tables
    layers = runner.target.attention_layers()
    kmax = layers[0].max_model_len
    ksc = layers[0].k_scale
    vsc = layers[0].v_scale

    def launch_all():
        for a in layers:
            hv.ops.verify_attention(q, a.k_cache, a.v_cache, bt, cu_q, cu_k, R, kmax,
                                    g.head_dim ** -0.5, k_scale=ksc, v_scale=vsc)

    # one verify step's worth of attention launches (36 layers) as a HIP graph, so
    # the timing is GPU time, as in the graph-replayed verify step
    us = graph_time_us(torch, dev, launch_all, reps) / len(layers)
    kv_bytes = L * g.num_kv_heads * g.head_dim * 2 * runner.kv.element_size()
    qo_bytes = 2 * R * g.num_heads * g.head_dim * 2
    per_launch = kv_bytes + qo_bytes
    achieved = per_launch / (us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 5), "traffic": None,
            "kernel": f"k_verify_attn<{'true' if runner.kv.element_size() == 1 else 'false'}, "
                      f"{g.num_heads // g.num_kv_heads}> (+ k_attn_combine when split)",
            "bytes_per_launch": per_launch, "avg_launch_us": round(us, 3),
            "shape": f"B=1 q={R} Hq={g.num_heads} Hkv={g.num_kv_heads} D={g.head_dim} L={L}",
            "launches": reps * len(layers)}


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default="spec", choices=["spec", "accept", "attention"])
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--gamma", type=int, default=3)
    ap.add_argument("--mode", default="reference", choices=["reference", "filtered", "greedy"])
    ap.add_argument("--logits", default="bf16", choices=["bf16", "f32"])
    ap.add_argument("--per-seq", action="store_true")
    ap.add_argument("--temperature", type=float, default=0.6)
    ap.add_argument("--top-k", type=int, default=0)
    ap.add_argument("--top-p", type=float, default=1.0)
    ap.add_argument("--draft", default="qwen3-0.6b", choices=["qwen3-0.6b", "forced"])
    ap.add_argument("--kv", default="auto", choices=["auto", "fp8"])
    ap.add_argument("--eager", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; the verify path shards "
                          "by sequence / KV head across GPUs by design but no multi-GPU run "
                          "is part of it", "n_gpus": args.gpus}))
        return 2
    if args.steps is None:
        args.steps = 96 if args.workload == "spec" else 200
    if args.warmup is None:
        args.warmup = 8 if args.workload == "spec" else 20
    import torch
    hv = importlib.import_module("hilda-vllm_amd")
    if args.workload == "spec":
        res = bench_spec(args, torch, hv)
    elif args.workload == "attention":
        res = bench_attention(args, torch, hv)
    else:
        res = bench_accept(args, torch, hv)
    print(json.dumps(res))
    return 0


if __name__ == "__main__":
    sys.exit(main())
