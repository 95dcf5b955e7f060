"""Paged-attention decode benchmark on one MI355X.

Workload (one "step" = one decode step of one attention layer for the whole
batch): Llama-3-8B-shape decode, batch 64, 32 q heads / 8 KV heads (GQA 4),
head_dim 128, block_size 16, every context 4096 tokens, bf16 KV in a
shuffled pool of 1.25x the blocks needed, q/K/V ~ N(0,1) (synthetic,
seeded).  Two pool copies are rotated between steps so the 256 MiB
Infinity Cache cannot serve a re-timed step.

Prints one JSON line: value = GB/s of algorithmic bytes (KV read once +
q read + out write + block tables + seq_lens) per step over the timed
steps; tok/s = batch / step time; roofline of the decode step against 8 TB/s;
cpu_baseline = the oracle's multithreaded fp32 decode on the host cores over
a bounded sample (4 of the 64 sequences).
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "truellm-engine_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

HBM_PEAK_GBS = 8000.0
METRIC = "paged-attn decode GB/s (% HBM peak) + tok/s, B=64 ctx4k, fp16 & KIVI-INT4 KV"


def algorithmic_bytes(S, H, n_kv, D, BS, lens, elem):
    kv = sum(lens) * n_kv * D * 2 * elem
    qo = S * H * D * elem * 2
    tables = sum((L + BS - 1) // BS for L in lens) * 4 + 4 * S
    return kv + qo + tables


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--partition-tokens", type=int, default=0)
    p.add_argument("--dtype", default="bf16", choices=["bf16", "fp16"])
    p.add_argument("--cpu-seconds", type=float, default=15.0)
    p.add_argument("--no-cpu", action="store_true")
    return p.parse_args()


def cpu_baseline(seconds, S_sample, H, n_kv, D, BS, L, threads):
    import numpy as np

    import inputs
    import oracle_lib as orc

    lens = [L] * S_sample
    case = inputs.make_paged_case(inputs.SEEDS[1], S_sample, H, n_kv, D, BS, lens, orc.BF16)
    nbytes = algorithmic_bytes(S_sample, H, n_kv, D, BS, lens, 2)
    reps, t_total = 0, 0.0
    while t_total < seconds or reps < 2:
        t0 = time.perf_counter()
        orc.paged_attention_f32(case.q, orc.BF16, case.k_cache, case.v_cache, orc.BF16,
                                case.tables, case.seq_lens, n_kv, case.scale, orc.GROUPED,
                                threads=threads)
        t_total += time.perf_counter() - t0
        reps += 1
    per = t_total / reps
    return {
        "value": round(nbytes / per / 1e9, 3),
        "unit": "GB/s",
        "tok_s": round(S_sample / per, 2),
        "cores": threads,
        "kind": "port",
        "sample": f"{S_sample} of the 64 sequences (ctx {L}, 32/8 heads, d 128, bf16 pool), "
                  f"{reps} runs of the oracle's fp32 pthread decode, {per * 1e3:.1f} ms each",
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1"}))
        sys.exit(2)

    import torch

    import tl_attn as tla

    torch.cuda.set_device(0)
    S, H, n_kv, D, BS, L = 64, 32, 8, 128, 16, 4096
    tdt = torch.bfloat16 if args.dtype == "bf16" else torch.float16
    nb = L // BS
    N = math.ceil(1.25 * S * nb)
    g = torch.Generator(device="cuda").manual_seed(0x7E5E0002)
    pools = []
    for _ in range(2):
        k = torch.randn(N, n_kv, D, BS, generator=g, device="cuda", dtype=tdt)
        v = torch.randn(N, n_kv, D, BS, generator=g, device="cuda", dtype=tdt)
        perm = torch.randperm(N, generator=g, device="cuda").to(torch.int32)
        tables = perm[: S * nb].view(S, nb).contiguous()
        pools.append((k, v, tables))
    q = torch.randn(S, H, D, generator=g, device="cuda", dtype=tdt)
    sl = torch.full((S,), L, dtype=torch.int32, device="cuda")
    out = torch.empty_like(q)
    scale = 1.0 / math.sqrt(D)
    desc = tla.make_decode_desc(q, pools[0][0], pools[0][2], n_kv, scale,
                                gqa_map=tla.GQA_GROUPED, partition_tokens=args.partition_tokens)
    ws = torch.empty(max(16, tla.workspace_bytes(desc, L)), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream()

    def step(i):
        k, v, tables = pools[i % 2]
        tla.paged_attention_decode(desc, out, q, k, v, tables, sl, L, ws, stream)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    ev[0].record(stream)
    for i in range(args.steps):
        step(i)
        ev[i + 1].record(stream)
    torch.cuda.synchronize()
    per_step = [ev[i].elapsed_time(ev[i + 1]) for i in range(args.steps)]
    total_ms = ev[0].elapsed_time(ev[-1])
    ms = total_ms / args.steps
    nbytes = algorithmic_bytes(S, H, n_kv, D, BS, [L] * S, 2)
    gbs = nbytes / (ms * 1e-3) / 1e9
    avg_launch_ms = sum(per_step) / len(per_step)
    achieved = nbytes / (avg_launch_ms * 1e-3) / 1e9

    res = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic",
        "config": {
            "workload": "paged-attention decode, Llama-3-8B shape",
            "batch": S, "q_heads": H, "kv_heads": n_kv, "head_dim": D, "block_size": BS,
            "context": L, "kv_dtype": args.dtype, "pool_blocks": N, "pools_rotated": 2,
            "partition_tokens": args.partition_tokens or "auto",
        },
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "tok_s": round(S / (ms * 1e-3), 1),
        "tok_s_32_layers": round(S / (ms * 1e-3) / 32, 1),
        "roofline": {
            "kernel": "paged decode step (decode_kernel + lse_reduce_kernel)",
            "bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
            "bytes_per_launch": nbytes, "traffic": None,
        },
    }
    if not args.no_cpu:
        threads = min(16, os.cpu_count() or 1)
        res["cpu_baseline"] = cpu_baseline(args.cpu_seconds, 4, H, n_kv, D, BS, L, threads)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
