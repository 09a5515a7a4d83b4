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
  accept  - the fused acceptance step at the batch-1 verify shape of the
            8B-target / 0.6B-draft run: B=1, gamma=3, V=151936, bf16 target
            logits (LM-head output) and f32 draft probabilities, T=0.6.
            One step = one hs_spec_accept call (row statistics + resample).
            Inputs rotate over enough copies to exceed the 256 MB MALL, so
            every step reads from HBM.
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


def _accept_inputs(torch, hv, dev, copies: int, gamma: int = 3, T: float = 0.6):
    w = hv.synthetic.accept_workload(1, gamma, seed=0, dtype="bf16", temperature=T)
    lg = torch.from_numpy(w["logits_bits"].view("int16")).to(dev).view(torch.bfloat16)
    q = torch.from_numpy(w["draft_probs"]).to(dev)
    bufs = [(lg.clone(), q.clone()) for _ in range(copies)]
    small = {k: torch.from_numpy(w[k]).to(dev)
             for k in ["draft_tokens", "temperatures", "u_accept", "u_resample"]}
    return w, bufs, small


def bench_accept(args, torch, hv):
    dev = torch.device("cuda:0")
    gamma = 3
    step_bytes = (gamma + 1) * V * 2 + gamma * V * 4  # bf16 target rows + f32 draft rows
    copies = max(2, int(512e6 // step_bytes) + 1)
    w, bufs, s = _accept_inputs(torch, hv, dev, copies, gamma)

    def step(i):
        lg, q = bufs[i % copies]
        return hv.ops.spec_accept(lg, q, s["draft_tokens"], s["temperatures"], s["u_accept"],
                                  s["u_resample"], mode="reference")

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for i in range(args.steps):
        out = step(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev0.elapsed_time(ev1)
    us_per_step = gpu_ms * 1e3 / args.steps
    nacc = int(out[0][0])
    achieved = step_bytes / (us_per_step * 1e-6) / 1e9
    res = {
        "metric": METRIC,
        "value": round(us_per_step, 3),
        "unit": "us/step (fused acceptance)",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_per_step / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 logits, f32 math",
        "data": "synthetic (seeded N(0,2^2) logits, draft = target + N(0,1))",
        "config": {"workload": "fused acceptance, B=1 gamma=3 V=151936 (config-3 verify shape)",
                   "batch": 1, "gamma": gamma, "vocab": V, "temperature": 0.6,
                   "mode": "reference", "input_copies_rotated": copies},
        "accepted_in_last_step": nacc,
        "wall_s": round(wall, 3),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": None, "bytes_per_step": step_bytes,
                     "kernels": "k_chunk_stats + k_sample_part + k_sample_final (one hs_spec_accept call)"},
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline_accept(torch, w, args.cpu_seconds)
    return res


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

    launch_all()
    torch.cuda.synchronize()
    # one verify step's worth of attention launches (36 layers) as a HIP graph, so
    # the timing is GPU time, as in the graph-replayed verify step
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            launch_all()
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
    us = e0.elapsed_time(e1) * 1e3 / (reps * len(layers))
    kv_bytes = L * g.num_kv_heads * g.head_dim * 2 * runner.kv.element_size()
    qo_bytes = 2 * R * g.num_heads * g.head_dim * 2
    per_launch = kv_bytes + qo_bytes
    achieved = per_launch / (us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 5), "traffic": None,
            "kernel": "k_verify_attn (+ k_attn_combine when split)",
            "bytes_per_launch": per_launch, "avg_launch_us": round(us, 3),
            "shape": f"B=1 q={R} Hq={g.num_heads} Hkv={g.num_kv_heads} D={g.head_dim} L={L}",
            "launches": reps * len(layers)}


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default="spec", choices=["spec", "accept"])
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
    else:
        res = bench_accept(args, torch, hv)
    print(json.dumps(res))
    return 0


if __name__ == "__main__":
    sys.exit(main())
