"""Paged-attention decode benchmark on one MI355X.

One "step" is one decode step of one attention layer for the whole batch.
Workloads (synthetic, seeded; q/K/V ~ N(0,1)):
  * headline: Llama-3-8B-shape decode, batch 64, 32 q heads / 8 KV heads
    (GQA 4), head_dim 128, block_size 16, every context 4096 tokens, bf16 KV
    in a shuffled pool of 1.25x the blocks needed;
  * the same shape with fp16 KV (the reference for the KIVI speed-up);
  * KIVI INT4 at the same shape: per-channel K / per-token V groups of 32,
    fp16 residual window of 128+ tokens, 4 outlier K channels per kv head
    scaled x8; each step appends one token per sequence (fp16 write plus
    quantise-on-append when a page completes) and then decodes.
Two copies of every pool are rotated between steps so the 256 MiB Infinity
Cache cannot serve a re-timed step.

The --steps timed steps are captured into one HIP graph, as a serving decode
loop runs (warmup steps run eagerly); after untimed replays bring the GPU to
its sustained clocks the graph is replayed R times (R >= 5, at least 60
steps in all), each replay timed with events on the replay stream, and a
workload's ms per step is the median replay's.

Prints one JSON line.  value = GB/s of algorithmic bytes (KV read once + q
read + out write + block tables + seq_lens) per bf16 step; roofline = the
same bytes over the decode launch's duration (one launch per step) against
8 TB/s; cpu_baseline = the oracle's fp32 decode on the host cores over a
bounded sample, one thread and all the cores of the GPU's CPU share.
"""
import argparse
import itertools
import json
import math
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "truellm-engine_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

HBM_PEAK_GBS = 8000.0
METRIC = "paged-attn decode GB/s (% HBM peak) + tok/s, B=64 ctx4k, fp16 & KIVI-INT4 KV"
S, H, NKV, D, BS, CTX = 64, 32, 8, 128, 16, 4096
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "decode_bf16_b64_ctx4096_hbm_traffic.md")


def algorithmic_bytes(lens, elem):
    """K+V read once, q read and out written, the block-table entries used
    and seq_lens."""
    kv = sum(lens) * NKV * D * 2 * elem
    qo = len(lens) * H * D * elem * 2
    tables = sum((L + BS - 1) // BS for L in lens) * 4 + 4 * len(lens)
    return kv + qo + tables


def config2b_lens():
    """Batch 64, lengths uniform in [512, 8192] (seed 0x7E5E0002)."""
    import numpy as np
    return np.random.default_rng(0x7E5E0002).integers(512, 8193, size=S).tolist()


def kivi_bytes(lens, R, completes_page, bits=4):
    """KIVI bytes of one step: pages (INT4: 160 B/token/kv head, INT8: 288)
    + fp16 window (512 B/token/kv head) + q/out + tables, plus the appended
    token and, for each sequence whose append completes a page, its
    quantisation (32 fp16 tokens read, one page of 5 KiB (INT4) or 9 KiB
    (INT8) written per kv head)."""
    page = 5120 if bits == 4 else 9216
    tot = 0
    for L, done in zip(lens, completes_page):
        lq = 0 if L <= R else ((L - R) // 32) * 32
        tot += NKV * (lq * (page // 32) + (L - lq) * 512)
        tot += (lq // 32 + (L - lq + BS - 1) // BS) * 4 + 4
        if done:
            tot += NKV * (32 * 512 + page)
    tot += len(lens) * H * D * 2 * 2
    tot += len(lens) * NKV * D * 2 * 2
    return tot


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--partition-tokens", type=int, default=0)
    p.add_argument("--cpu-seconds", type=float, default=15.0)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--only", default="all", choices=["all", "bf16", "fp16", "kivi", "fp8", "config2b", "v2",
                                                     "prefill", "blocks", "rope", "vq", "norm"])
    p.add_argument("--block-size", type=int, default=16, choices=[8, 16, 32, 64, 128, 256],
                   help="block size of the bf16 / fp16 / FP8 decode pools (with --only bf16, fp16 or fp8; "
                        "FP8 from 16)")
    p.add_argument("--no-graph", action="store_true",
                   help="launch the timed steps eagerly (for counter passes that cannot follow graphs)")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only run a plain 1 GiB device-to-device copy 5 times (HBM byte counters of a "
                        "kernel of known traffic) and exit")
    return p.parse_args()


USE_GRAPH = True


WARM_MS = 30.0


POOL_ARENA = {}


def pool_buffer(name, shape, dtype, g, index=0):
    """A KV pool of the given shape and dtype, N(0, 1) from generator g, in a
    device buffer allocated once for the whole run and shared by every
    workload (pools 'k0', 'v0', 'k1', 'v1'): the workloads then stream the
    same physical memory.  Pools allocated later in a run, after earlier
    workloads' memory had been freed, were up to 4 % slower for the same
    kernel (fp16 against bf16, the v2 operator against the library plan);
    main() allocates the arena first, at the largest size any workload
    needs."""
    import torch
    nbytes = math.prod(shape) * torch.empty((), dtype=dtype).element_size()
    off = index * ((nbytes + 4095) // 4096 * 4096)      # pool `index` of this arena
    buf = POOL_ARENA.get(name)
    if buf is None or buf.numel() < off + nbytes:
        buf = torch.empty(off + nbytes, dtype=torch.uint8, device="cuda")
        POOL_ARENA[name] = buf
    t = buf[off:off + nbytes].view(dtype).view(shape)
    if dtype in (torch.float16, torch.bfloat16, torch.float32):
        t.normal_(0.0, 1.0, generator=g)
    return t


def arena_bytes():
    """Bytes of the largest pool any workload uses (per pool)."""
    blocks_2a = math.ceil(1.25 * S * (CTX // BS))
    blocks_2b = math.ceil(1.25 * sum((L + BS - 1) // BS for L in config2b_lens()))
    blocks_kivi = S * ((CTX + 32 + 256 + BS - 1) // BS) + 8
    return max(blocks_2a, blocks_2b, blocks_kivi) * NKV * D * BS * 2


MIN_TIMED_STEPS, MIN_REPLAYS = 60, 5
SPREAD = {}      # workload -> (min, max) ms per step over the timed replays


def timed(step, steps, warmup, name=None):
    """Run `warmup` eager steps, capture the next `steps` steps into one HIP
    graph, replay it untimed until about WARM_MS of GPU work has run, then
    time R = max(5, ceil(60 / steps)) replays one by one with events on the
    replay stream.  Returns the median replay's ms per step (the spread goes
    to SPREAD[name]).  A serving decode loop runs the same way: the graph
    removes the per-launch host cost, which otherwise exceeds a short step's
    GPU time, and the GPU runs at the clocks of sustained load (from an idle
    GPU the first ~10 ms of the KIVI decode ran up to 10 % slower)."""
    import statistics

    import torch
    stream = torch.cuda.current_stream()
    for i in range(warmup):
        step(i, stream)
    torch.cuda.synchronize()
    reps = max(MIN_REPLAYS, -(-MIN_TIMED_STEPS // steps))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    per = []
    if not USE_GRAPH:
        for _ in range(reps):
            e0.record(stream)
            for i in range(steps):
                step(warmup + i, stream)
            e1.record(stream)
            torch.cuda.synchronize()
            per.append(e0.elapsed_time(e1) / steps)
    else:
        graph = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream()
        with torch.cuda.graph(graph, stream=cap):
            for i in range(steps):
                step(warmup + i, cap)
        e0.record(stream)
        graph.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        for _ in range(min(50, int(WARM_MS / max(e0.elapsed_time(e1), 1e-3)))):
            graph.replay()
        torch.cuda.synchronize()
        for _ in range(reps):
            e0.record(stream)
            graph.replay()
            e1.record(stream)
            torch.cuda.synchronize()
            per.append(e0.elapsed_time(e1) / steps)
    if name:
        SPREAD[name] = (min(per), max(per), reps, steps)
    return statistics.median(per)


def bench_decode(args, dtype, append=False, lens=None, partition_tokens=None, v2=False, name=None, layers=2,
                 v2_capacity=None):
    """Decode of one layer over the given lengths (default: batch 64, every
    context 4096) with the library plan (or partition_tokens), through
    tl_paged_attention_decode or, with v2, the reference-named
    tl_paged_attention_v2 on the engine's scratch sizes.  With append, every
    step first writes each sequence's newest token (position L - 1) into the
    pool with reshape_and_cache, as an engine's decode step does before
    attention: the fp16 counterpart of the KIVI step, whose append is fused
    into its launch.  Step i reads pool i % layers (layers pools of their
    own, as the layers of a model keep theirs)."""
    import torch

    import tl_attn as tla


    lens = [CTX] * S if lens is None else list(lens)
    B = len(lens)
    pt = args.partition_tokens if partition_tokens is None else partition_tokens
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    nbs = [(L + BS - 1) // BS for L in lens]
    mb = max(nbs)
    N = math.ceil(1.25 * sum(nbs))
    g = torch.Generator(device="cuda").manual_seed(0x7E5E0002)
    pools = []
    for li in range(layers):
        k = pool_buffer(f"k{li % 2}", (N, NKV, D, BS), tdt, g, li // 2)
        v = pool_buffer(f"v{li % 2}", (N, NKV, D, BS), tdt, g, li // 2)
        perm = torch.randperm(N, generator=g, device="cuda").to(torch.int32).cpu()
        tables = torch.full((B, mb), -1, dtype=torch.int32)
        off = 0
        for s_, nb in enumerate(nbs):
            tables[s_, :nb] = perm[off:off + nb]
            off += nb
        pools.append((k, v, tables.cuda()))
    q = torch.randn(B, H, D, generator=g, device="cuda", dtype=tdt)
    sl = torch.tensor(lens, dtype=torch.int32, device="cuda")
    max_ctx = max(lens)
    out = torch.empty_like(q)
    scale = 1.0 / math.sqrt(D)
    desc = tla.make_decode_desc(q, pools[0][0], pools[0][2], NKV, scale, gqa_map=tla.GQA_GROUPED, partition_tokens=pt)
    ws = torch.empty(max(16, tla.workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
    if v2:
        # v2_capacity: the scratch allocated for that many partitions (the
        # engine sizes it for its training context) and passed through
        # tl_paged_attention_v2_capacity
        P = tla.v2_num_partitions(max_ctx, BS) if v2_capacity is None else v2_capacity
        v2_parts, v2_pt = tla.v2_plan(B, H, NKV, D, BS, tla.dtype_code(q), max_ctx, scratch_partitions=v2_capacity)
        es = torch.empty(B, H, P, dtype=torch.float32, device="cuda")
        ml = torch.empty_like(es)
        tmp = torch.empty(B, H, P, D, dtype=tdt, device="cuda")

    if append:
        knew = torch.randn(B, NKV, D, generator=g, device="cuda", dtype=tdt)
        vnew = torch.randn(B, NKV, D, generator=g, device="cuda", dtype=tdt)
        pos = sl.long() - 1
        rows = torch.arange(B, device="cuda")
        slots = [(tables[rows, pos // BS] * BS + pos % BS).to(torch.int32).contiguous() for _k, _v, tables in pools]

    def step(i, stream):
        k, v, tables = pools[i % layers]
        if append:
            tla.reshape_and_cache_split(knew, vnew, k, v, slots[i % layers], stream)
        if v2:
            tla.paged_attention_v2(out, es, ml, tmp, q, k, v, tables, sl, NKV, scale, D, BS, max_ctx, stream,
                                   gqa_map=tla.GQA_GROUPED, scratch_partitions=v2_capacity)
        else:
            tla.paged_attention_decode(desc, out, q, k, v, tables, sl, max_ctx, ws, stream)

    ms = timed(step, max(args.steps, layers), args.warmup, name)
    nbytes = algorithmic_bytes(lens, 2)
    parts = max(1, tla.workspace_bytes(desc, max_ctx) // (B * H * (D + 2) * 4))
    return {
        "ms_per_step": ms, "gbs": nbytes / (ms * 1e-3) / 1e9, "tok_s": B / (ms * 1e-3),
        "bytes": nbytes, "launch_ms": ms, "pool_blocks": N,            # one decode launch per step
        "workspace_bytes": tla.workspace_bytes(desc, max_ctx),
        "partitions": v2_parts if v2 else parts,
        "partition_tokens": v2_pt if v2 else (-(-max_ctx // parts) if parts == 1 else None),
        "pool_bytes_all_layers": 2 * N * NKV * D * BS * 2 * layers,
    }


def kivi_steps(steps):
    """Timed KIVI steps: a whole number of 64, so that each of the two pool
    replicas (alternating steps) appends 32 tokens per 64 steps and its fp16
    window runs through every length of its cycle (128 .. 159 tokens, one
    page build) -- the window's length changes the step time, so a partial
    cycle would not be the sustained rate."""
    return max(64, (steps + 63) // 64 * 64)


def bench_kivi(args, R=128, mixed=False, name=None, bits=4, pre_rope=False, build_ahead=False):
    """KIVI append + decode steps (INT4 pages, or INT8 with bits=8) at batch
    64 from context 4096 (mixed: sequence s starts at 4096 + s mod 32 tokens,
    so two sequences complete a page at every step instead of all 64 on one
    step in 32).  pre_rope: keys held before RoPE, each rotated at its
    position inside attention (fp32 tables of 8192 positions).  build_ahead:
    each page written in eighths by the 8 steps before the one that
    completes it (the page tables are set up front)."""
    import torch

    import tl_attn as tla


    n_timed = kivi_steps(args.steps)
    total_steps = args.warmup + n_timed
    L0 = [CTX + (s_ % 32 if mixed else 0) for s_ in range(S)]
    Lmax = max(L0) + total_steps
    nb = (Lmax + BS - 1) // BS
    N = S * nb + 8
    max_pages = Lmax // 32 + 1
    g = torch.Generator(device="cuda").manual_seed(0x7E5E0003)
    reps = []
    for _ in range(2):
        k = pool_buffer(f"k{len(reps)}", (N, NKV, D, BS), torch.float16, g)
        v = pool_buffer(f"v{len(reps)}", (N, NKV, D, BS), torch.float16, g)
        for h in range(NKV):                                  # 4 outlier K channels x8
            ch = torch.randperm(D, generator=g, device="cuda")[:4]
            k[:, h, ch, :] *= 8
        perm = torch.randperm(N, generator=g, device="cuda").to(torch.int32)
        tables = perm[: S * nb].view(S, nb).contiguous()
        num_pages = S * max_pages + 8
        pperm = torch.randperm(num_pages, generator=g, device="cuda").to(torch.int32)
        ptables = pperm[: S * max_pages].view(S, max_pages).contiguous()
        pages = torch.zeros(num_pages, NKV, tla.kivi_page_bytes(bits), dtype=torch.uint8, device="cuda")
        reps.append([k, v, tables, ptables, pages, num_pages])
    q = torch.randn(S, H, D, generator=g, device="cuda", dtype=torch.float16)
    knew = torch.randn(S, NKV, D, generator=g, device="cuda", dtype=torch.float16)
    vnew = torch.randn(S, NKV, D, generator=g, device="cuda", dtype=torch.float16)
    out = torch.empty_like(q)
    scale = 1.0 / math.sqrt(D)
    # per replica: the lengths after each of its appends, slots of the new tokens
    lens_host = {0: list(L0), 1: list(L0)}
    plan = []
    for i in range(total_steps):
        r = i % 2
        lens_host[r] = [L + 1 for L in lens_host[r]]
        plan.append((r, list(lens_host[r])))
    sl_dev, slot_dev = [], []
    tables_host = [rep[2].cpu() for rep in reps]
    rows = torch.arange(S)
    for r, lens in plan:
        lt = torch.tensor(lens, dtype=torch.int64)
        sl_dev.append(lt.to(torch.int32).cuda())
        pos = lt - 1
        slot = tables_host[r][rows, pos // BS] * BS + pos % BS
        slot_dev.append(slot.to(torch.int32).cuda())
    desc0 = tla.make_kivi_desc(q, reps[0][0], reps[0][2], reps[0][3], reps[0][5], NKV, scale,
                               residual_length=R, gqa_map=tla.GQA_GROUPED, bits=bits)
    ws = torch.empty(max(16, tla.kivi_workspace_bytes(desc0, Lmax)), dtype=torch.uint8, device="cuda")
    for rep in reps:
        d = tla.make_kivi_desc(q, rep[0], rep[2], rep[3], rep[5], NKV, scale, residual_length=R, bits=bits,
                               build_ahead=build_ahead)
        sl0 = torch.tensor(L0, dtype=torch.int32, device="cuda")
        tla.kivi_build_pages(d, rep[0], rep[1], rep[2], sl0, rep[3], rep[4], max(L0))
    descs = [tla.make_kivi_desc(q, rep[0], rep[2], rep[3], rep[5], NKV, scale, residual_length=R, bits=bits,
                                pre_rope_keys=pre_rope, build_ahead=build_ahead) for rep in reps]
    if pre_rope:
        i = torch.arange(D // 2, dtype=torch.float32)
        theta = torch.arange(8192, dtype=torch.float32)[:, None] / torch.pow(10000.0, 2.0 * i / D)
        cos_t, sin_t = torch.cos(theta).cuda(), torch.sin(theta).cuda()

    def step(i, stream):
        r, lens = plan[i]
        k, v, tables, ptables, pages, _ = reps[r]
        if pre_rope:
            tla.kivi_decode_step_pre_rope(descs[r], out, q, knew, vnew, slot_dev[i], pages, ptables, k, v, tables,
                                          sl_dev[i], max(lens), cos_t, sin_t, tla.ROPE_HALVES, ws, stream)
        else:
            tla.kivi_decode_step(descs[r], out, q, knew, vnew, slot_dev[i], pages, ptables, k, v, tables,
                                 sl_dev[i], max(lens), ws, stream)

    ms = timed(step, n_timed, args.warmup, name)
    lq = lambda x: 0 if x <= R else ((x - R) // 32) * 32
    nbytes = [kivi_bytes(lens, R, [lq(L) > lq(L - 1) for L in lens], bits) for _, lens in plan[args.warmup:]]
    avg_bytes = sum(nbytes) / len(nbytes)
    return {"ms_per_step": ms, "gbs": avg_bytes / (ms * 1e-3) / 1e9, "tok_s": S / (ms * 1e-3),
            "bytes_per_step": avg_bytes, "residual_length": R, "group": 32, "steps": n_timed,
            "build_ahead": int(bool(build_ahead))}


F8_S, F8_CTX = 16, 32768


def bench_rope(args):
    """The write side of one decode step at batch 64 (Llama-3-8B shape):
    RoPE (adjacent pairs, fp32 tables [8192, 64]) on q [64, 32, 128] and k
    [64, 8, 128], then k and v into the bf16 pools, one launch."""
    import torch

    import tl_attn as tla


    g = torch.Generator(device="cuda").manual_seed(0x7E5E0007)
    N = S * (CTX // BS + 1)
    q = torch.randn(S, H, D, generator=g, device="cuda", dtype=torch.bfloat16)
    k = torch.randn(S, NKV, D, generator=g, device="cuda", dtype=torch.bfloat16)
    v = torch.randn(S, NKV, D, generator=g, device="cuda", dtype=torch.bfloat16)
    kc = torch.zeros(N, NKV, D, BS, device="cuda", dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    # sequence s owns ctx/bs + 1 blocks of the pool in a random order (as an
    # allocator's free list hands them out), and position ctx lands in its last
    nbs = CTX // BS + 1
    tables = torch.randperm(N, generator=g, device="cuda").to(torch.int32).view(S, nbs).contiguous()
    slots = (tables[:, CTX // BS] * BS + CTX % BS).contiguous()
    pos = torch.full((S,), CTX, device="cuda", dtype=torch.int32)
    i = torch.arange(D // 2, device="cuda", dtype=torch.float32)
    theta = torch.arange(8192, device="cuda", dtype=torch.float32)[:, None] / torch.pow(10000.0, 2 * i / D)
    cos_t, sin_t = torch.cos(theta).contiguous(), torch.sin(theta).contiguous()
    q_out = torch.empty_like(q)

    def step(i_, stream):
        tla.rope_reshape_and_cache(q, k, v, kc, vc, slots, pos, cos_t, sin_t, tla.ROPE_ADJACENT, q_out=q_out,
                                   stream=stream)

    ms = timed(step, args.steps, args.warmup)
    nbytes = 2 * q.numel() * 2 + 4 * k.numel() * 2 + 2 * S * (D // 2) * 4 + 2 * S * 4
    # the append's full cost shows in the decode that follows it (lines the
    # append left partly written are written back during the decode): the
    # append + decode step against the decode alone, over the same pools
    # (ctx + 1 tokens per sequence)
    sl = torch.full((S,), CTX + 1, dtype=torch.int32, device="cuda")
    out = torch.empty_like(q)
    desc = tla.make_decode_desc(q_out, kc, tables, NKV, 1.0 / math.sqrt(D), gqa_map=tla.GQA_GROUPED,
                                partition_tokens=-1)

    def decode(i_, stream):
        tla.paged_attention_decode(desc, out, q_out, kc, vc, tables, sl, CTX + 1, None, stream)

    def both(i_, stream):
        step(i_, stream)
        decode(i_, stream)

    ms_d = timed(decode, args.steps, args.warmup)
    ms_b = timed(both, args.steps, args.warmup)
    return {"us": ms * 1e3, "bytes": nbytes, "us_decode": ms_d * 1e3, "us_append_then_decode": ms_b * 1e3}


NA_ROWS, NA_HID, NA_FFN = 4096, 4096, 14336


def bench_norm_act(args):
    """A 4096-token prefill chunk of Llama-3-8B's layer edges, bf16:
    fused_add_rms_norm over [4096, 4096] (read x and the residual, write the
    residual and out) and silu_and_mul over [4096, 14336] (read gate and up,
    write out)."""
    import torch

    import tl_attn as tla


    g = torch.Generator(device="cuda").manual_seed(0x7E5E0009)
    x = torch.randn(NA_ROWS, NA_HID, generator=g, device="cuda", dtype=torch.bfloat16)
    res = torch.randn_like(x)
    w = torch.randn(NA_HID, generator=g, device="cuda", dtype=torch.bfloat16)
    out = torch.empty_like(x)
    gate = torch.randn(NA_ROWS, NA_FFN, generator=g, device="cuda", dtype=torch.bfloat16)
    up = torch.randn_like(gate)
    act = torch.empty_like(gate)

    def norm_step(i, stream):
        tla.fused_add_rms_norm(out, res, x, w, 1e-5, stream)

    def act_step(i, stream):
        tla.act_and_mul(act, gate, up, tla.ACT_SILU, stream)

    ms_n = timed(norm_step, args.steps, args.warmup)
    ms_a = timed(act_step, args.steps, args.warmup)
    bn = 4 * x.numel() * 2 + w.numel() * 2
    ba = 3 * gate.numel() * 2
    return {"norm_us": ms_n * 1e3, "norm_bytes": bn, "act_us": ms_a * 1e3, "act_bytes": ba}


VQ_N, VQ_K = 2048 * 8, 256


def bench_vq(args):
    """VQ encode of one 2048-token layer (8 kv heads, d 128: 16384 fp16
    vectors) against a 256-entry codebook: 3 fp32 flops (subtract, fma) per
    (vector, entry, dim), in the reference's exact order."""
    import torch

    import tl_attn as tla


    g = torch.Generator(device="cuda").manual_seed(0x7E5E0008)
    kv = torch.randn(VQ_N, D, generator=g, device="cuda", dtype=torch.float16)
    book = torch.randn(VQ_K, D, generator=g, device="cuda", dtype=torch.float16)
    idx = torch.zeros(VQ_N, dtype=torch.int16, device="cuda")

    def step(i, stream):
        tla.vq_encode(kv, book, idx, stream)

    ms = timed(step, max(4, args.steps // 5), max(2, args.warmup // 5))
    flops = 3 * VQ_N * VQ_K * D
    return {"ms": ms, "flops": flops, "tflops": flops / (ms * 1e-3) / 1e12}


CB_BLOCKS, CB_PAIRS = 8192, 2048


def bench_copy_blocks(args):
    """copy_blocks: 2048 (src, dst) pairs out of an 8192-block fp16 pool pair
    (8 kv heads, d 128, bs 16: 32 KiB per block and pool), the shape of a
    prefix-cache fork of 2048 blocks.  Bytes moved = 2 pools x pairs x block
    read + written."""
    import torch

    import tl_attn as tla


    g = torch.Generator(device="cuda").manual_seed(0x7E5E0006)
    k = torch.randn(CB_BLOCKS, NKV, D, BS, generator=g, device="cuda", dtype=torch.float16)
    v = torch.randn_like(k)
    perm = torch.randperm(CB_BLOCKS, generator=g, device="cuda")
    m = torch.stack([perm[:CB_PAIRS], perm[CB_PAIRS:2 * CB_PAIRS]], 1).to(torch.int32).contiguous()

    def step(i, stream):
        tla.copy_blocks(k, v, m, stream)

    ms = timed(step, args.steps, args.warmup)
    nbytes = 2 * 2 * CB_PAIRS * k[0].numel() * k.element_size()
    return {"ms": ms, "bytes": nbytes, "gbs": nbytes / (ms * 1e-3) / 1e9}


def bench_fp8(args, partition_tokens=0, name=None):
    """FP8 E4M3 KV long-context decode: batch 16, 32 q / 8 kv heads, d 128,
    bs 16, every context 32768, per-tensor fp32 scales absmax/448 (K/V drawn
    N(0,1) in fp16 and cast), bf16 q/out.  partition_tokens 0: the library's
    own split-K plan; 512: the 64 partitions of 512 tokens the workload
    names.  The log-sum-exp reduce is in the timed step."""
    import torch

    import tl_attn as tla


    nb = F8_CTX // BS
    N = math.ceil(1.25 * F8_S * nb)
    g = torch.Generator(device="cuda").manual_seed(0x7E5E0004)
    pools = []
    for _ in range(2):
        kv = []
        for t_ in range(2):
            x = torch.randn(N, NKV, D, BS, generator=g, device="cuda", dtype=torch.float16)
            s = x.abs().max().float() / 448.0
            codes = pool_buffer(f"{'kv'[t_]}{len(pools)}", (N, NKV, D, BS), torch.uint8, g)
            for c0 in range(0, N, 4096):
                codes[c0:c0 + 4096].copy_((x[c0:c0 + 4096].float() / s).to(torch.float8_e4m3fn).view(torch.uint8))
            kv.append((codes, float(s)))
            del x
        perm = torch.randperm(N, generator=g, device="cuda").to(torch.int32)
        pools.append((kv[0], kv[1], perm[: F8_S * nb].view(F8_S, nb).contiguous()))
    q = torch.randn(F8_S, H, D, generator=g, device="cuda", dtype=torch.bfloat16)
    sl = torch.full((F8_S,), F8_CTX, dtype=torch.int32, device="cuda")
    out = torch.empty_like(q)
    descs = []
    for (kq, ks), (vq, vs), tables in pools:
        descs.append(tla.make_decode_desc(q, kq, tables, NKV, 1.0 / math.sqrt(D), gqa_map=tla.GQA_GROUPED,
                                          partition_tokens=partition_tokens, k_scale=ks, v_scale=vs))
    ws = torch.empty(max(16, tla.workspace_bytes(descs[0], F8_CTX)), dtype=torch.uint8, device="cuda")

    def step(i, stream):
        (kq, _), (vq, _), tables = pools[i % 2]
        tla.paged_attention_decode(descs[i % 2], out, q, kq, vq, tables, sl, F8_CTX, ws, stream)

    ms = timed(step, args.steps, args.warmup, name)
    kv_bytes = F8_S * F8_CTX * NKV * D * 2
    nbytes = kv_bytes + F8_S * H * D * 2 * 2 + F8_S * nb * 4 + F8_S * 4
    P = max(1, tla.workspace_bytes(descs[0], F8_CTX) // (F8_S * H * (D + 2) * 4))
    part = F8_S * H * P * (D + 2) * 4 * 2
    return {"ms_per_step": ms, "gbs": nbytes / (ms * 1e-3) / 1e9, "tok_s": F8_S / (ms * 1e-3),
            "bytes": nbytes, "partial_bytes": part, "partitions": P}


PF_H, PF_NKV, PF_SEQS, PF_PROMPT, PF_CHUNK, PF_DEC, PF_DEC_L = 64, 8, 8, 2048, 512, 32, 2048


def prefill_flops():
    """4 d multiply-add FLOPs per unmasked (query, key) pair, QK^T plus PV,
    over the 4 causal chunks of every prompt and every q head."""
    per_head = 0
    for c in range(PF_PROMPT // PF_CHUNK):
        per_head += 4 * D * (PF_CHUNK * PF_CHUNK * c + PF_CHUNK * (PF_CHUNK + 1) // 2)
    return per_head * PF_H * PF_SEQS


def bench_prefill(args):
    """Chunked prefill, Llama-3-70B attention shape (64 q / 8 kv heads, d 128,
    bf16): 8 prompts of 2048 tokens as 4 launches of 512-token causal chunks
    (chunk c sees the 512 c tokens before it), every launch also carrying 32
    decode rows at context 2048.  One step = the 4 launches."""
    import torch

    import tl_attn as tla


    S = PF_SEQS + PF_DEC
    nb = PF_PROMPT // BS
    N = math.ceil(1.25 * S * nb)
    g = torch.Generator(device="cuda").manual_seed(0x7E5E0005)
    pools = []
    for _ in range(2):
        k = pool_buffer(f"k{len(pools)}", (N, PF_NKV, D, BS), torch.bfloat16, g)
        v = pool_buffer(f"v{len(pools)}", (N, PF_NKV, D, BS), torch.bfloat16, g)
        perm = torch.randperm(N, generator=g, device="cuda").to(torch.int32)
        pools.append((k, v, perm[: S * nb].view(S, nb).contiguous()))
    nq = PF_SEQS * PF_CHUNK + PF_DEC
    q = torch.randn(nq, PF_H, D, generator=g, device="cuda", dtype=torch.bfloat16)
    out = torch.empty_like(q)
    q_lens = [PF_CHUNK] * PF_SEQS + [1] * PF_DEC
    cu = torch.tensor([0] + list(itertools.accumulate(q_lens)), dtype=torch.int32, device="cuda")
    lens = []
    for c in range(PF_PROMPT // PF_CHUNK):
        lens.append(torch.tensor([PF_CHUNK * (c + 1)] * PF_SEQS + [PF_DEC_L] * PF_DEC, dtype=torch.int32,
                                 device="cuda"))
    desc = tla.make_prefill_desc(q, pools[0][0], pools[0][2], S, PF_NKV, 1.0 / math.sqrt(D),
                                 num_prefill_seqs=PF_SEQS)

    def step(i, stream):
        k, v, tables = pools[i % 2]
        for c in range(PF_PROMPT // PF_CHUNK):
            tla.chunked_prefill(desc, out, q, cu, k, v, tables, lens[c], PF_CHUNK, stream)

    ms = timed(step, max(4, args.steps // 5), max(2, args.warmup // 5))
    flops = prefill_flops()
    dec_bytes = (PF_PROMPT // PF_CHUNK) * PF_DEC * PF_DEC_L * PF_NKV * D * 2 * 2
    return {"ms_per_step": ms, "tflops": flops / (ms * 1e-3) / 1e12, "flops": flops,
            "ms_per_launch": ms / (PF_PROMPT // PF_CHUNK), "decode_row_bytes": dec_bytes}


def traffic_from_profile():
    """HBM bytes per decode launch measured with rocprofv3 --pmc (FETCH_SIZE,
    WRITE_SIZE) and recorded in the profile summary, if present."""
    try:
        text = open(TRAFFIC_PROFILE).read()
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9]+)", text)
    return int(m.group(1)) if m else None


def cpu_info():
    """nproc, the CPUs this process may run on, the cores the GPU's share of
    the host gives it (OMP_NUM_THREADS where the host sets it) and the CPU
    model from lscpu."""
    import subprocess
    info = {"nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0))}
    share = os.environ.get("OMP_NUM_THREADS", "")
    info["threads_all_cores"] = min(int(share), info["affinity"]) if share.isdigit() and int(share) > 0 \
        else info["affinity"]
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        m = re.search(r"^Model name:\s*(.+)$", out, re.M)
        info["model"] = m.group(1).strip() if m else None
    except (OSError, subprocess.SubprocessError):
        info["model"] = None
    return info


def _median_time(fn, seconds, min_runs=5, warm=2):
    """Median wall time of fn() over at least min_runs runs (and about
    `seconds` in all) after `warm` untimed runs."""
    import statistics
    for _ in range(warm):
        fn()
    times = []
    while sum(times) < seconds or len(times) < min_runs:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def _host_u16(t):
    import numpy as np
    return t.contiguous().view(__import__("torch").int16).cpu().numpy().view(np.uint16)


def cpu_baseline(seconds):
    """The CPU path timed on the host cores beside the GPU, one entry per
    decode workload: the oracle's fp32 decode (threads over (sequence, kv
    head)) for the fp16 batch-4 workload (full size), the bf16 headline
    (full size) and the FP8 long-context step (full size), and its fp32
    paged-KIVI decode for the KIVI INT4 step (full size, one decode step).
    Each runs on all the cores of this GPU's CPU share over the whole batch
    and on one thread over a bounded sample of sequences; median of at least
    5 runs after 2 untimed ones.  Inputs are generated as the GPU lines'
    (same shapes, seeds and distributions; the large pools on the GPU, then
    copied to the host)."""
    import numpy as np
    import torch

    import inputs
    import oracle_lib as orc
    import tl_attn as tla

    info = cpu_info()
    ncore = info["threads_all_cores"]
    budget = max(0.5, seconds / 8)
    out = {}

    def entry(name, workload, nbytes_all, nbytes_one, n_one, S_all, run_all, run_one):
        ta, na = _median_time(run_all, budget)
        t1, n1 = _median_time(run_one, budget)
        out[name] = {
            "workload": workload,
            "all_cores": {"gbs": round(nbytes_all / ta / 1e9, 3), "tok_s": round(S_all / ta, 2),
                          "ms_per_step": round(ta * 1e3, 3), "runs": na, "threads": ncore},
            "single_thread": {"gbs": round(nbytes_one / t1 / 1e9, 3), "tok_s": round(n_one / t1, 2),
                              "ms_per_run": round(t1 * 1e3, 3), "runs": n1, "sequences": n_one},
        }

    # fp16 batch 4 (the reference CPU path's workload), full size
    lens1 = inputs.uniform_lens(inputs.SEEDS[0], 4, 128, 1024)
    c1 = inputs.make_paged_case(inputs.SEEDS[0], 4, H, NKV, D, 16, lens1, orc.F16, num_blocks=512, max_blocks=64)
    b1 = 4096 * int(lens1.sum()) + 4 * H * D * 2 * 2
    f1 = lambda th: (lambda: orc.paged_attention_f32(c1.q, orc.F16, c1.k_cache, c1.v_cache, orc.F16, c1.tables,
                                                     c1.seq_lens, NKV, c1.scale, orc.GROUPED, threads=th))
    entry("fp16_batch4", "fp16, batch 4, 32/8 heads, d 128, bs 16, lengths uniform in [128, 1024], 512-block pool",
          b1, b1, 4, 4, f1(ncore), f1(1))

    g = torch.Generator(device="cuda").manual_seed(inputs.SEEDS[1])

    def pools(nblocks, dtype):
        k = torch.randn(nblocks, NKV, D, 16, generator=g, device="cuda", dtype=torch.float32)
        v = torch.randn(nblocks, NKV, D, 16, generator=g, device="cuda", dtype=torch.float32)
        return k.to(dtype), v.to(dtype)

    # bf16 headline: batch 64, ctx 4096, full size
    nb = CTX // 16
    N = math.ceil(1.25 * S * nb)
    k, v = pools(N, torch.bfloat16)
    tab = torch.randperm(N, generator=g, device="cuda").to(torch.int32)[: S * nb].view(S, nb).cpu().numpy()
    q = _host_u16(torch.randn(S, H, D, generator=g, device="cuda").to(torch.bfloat16))
    kh, vh = _host_u16(k), _host_u16(v)
    del k, v
    lens2 = np.full(S, CTX, np.int32)
    n1 = 8
    sc = 1.0 / math.sqrt(D)
    f2 = lambda th, n: (lambda: orc.paged_attention_f32(q[:n], orc.BF16, kh, vh, orc.BF16, tab[:n], lens2[:n], NKV,
                                                        sc, orc.GROUPED, threads=th))
    entry("bf16_b64_ctx4096", "bf16, batch 64, ctx 4096, 32/8 heads, d 128, bs 16, shuffled 1.25x pool",
          algorithmic_bytes([CTX] * S, 2), algorithmic_bytes([CTX] * n1, 2), n1, S, f2(ncore, S), f2(1, n1))
    del kh, vh

    # KIVI INT4 at ctx 4096 (pages of the first 3968 tokens, the fp16 window
    # of the last 128), one decode step, full size
    R = 128
    L = CTX
    max_pages = (L + 32) // 32 + 1
    nbk = (L + 16 - 1) // 16 + 1
    N3 = S * nbk + 8
    k, v = pools(N3, torch.float16)
    for h in range(NKV):
        ch = torch.randperm(D, generator=g, device="cuda")[:4]
        k[:, h, ch, :] *= 8
    tab3 = torch.randperm(N3, generator=g, device="cuda").to(torch.int32)[: S * nbk].view(S, nbk).contiguous()
    num_pages = S * max_pages + 8
    ptab = torch.randperm(num_pages, generator=g, device="cuda").to(torch.int32)[: S * max_pages]
    ptab = ptab.view(S, max_pages).contiguous()
    pages = torch.zeros(num_pages, NKV, tla.kivi_page_bytes(4), dtype=torch.uint8, device="cuda")
    q3 = torch.randn(S, H, D, generator=g, device="cuda", dtype=torch.float16)
    sl3 = torch.full((S,), L, dtype=torch.int32, device="cuda")
    d3 = tla.make_kivi_desc(q3, k, tab3, ptab, num_pages, NKV, sc, residual_length=R, bits=4)
    tla.kivi_build_pages(d3, k, v, tab3, sl3, ptab, pages, L)
    torch.cuda.synchronize()
    kh, vh, q3h = _host_u16(k), _host_u16(v), _host_u16(q3)
    pg, pt3, t3 = pages.cpu().numpy(), ptab.cpu().numpy(), tab3.cpu().numpy()
    del k, v, pages
    lens3 = np.full(S, L, np.int32)
    kb = lambda n: kivi_bytes([L] * n, R, [False] * n) - n * NKV * D * 2 * 2   # no appended token
    f3 = lambda th, n: (lambda: orc.kivi_paged_attention_f32(q3h[:n], pg, pt3[:n], kh, vh, t3[:n], lens3[:n], NKV,
                                                             R, sc, orc.GROUPED, 4, threads=th))
    entry("kivi_int4_b64_ctx4096", "KIVI INT4 pages (G 32, R 128), batch 64, ctx 4096, 32/8 heads, one decode step "
          "(pages dequantised by the oracle's page routine, fp32 attention)",
          kb(S), kb(n1), n1, S, f3(ncore, S), f3(1, n1))
    del kh, vh, pg

    # FP8 E4M3, batch 16, ctx 32768, per-tensor absmax / 448 scales, full size
    nb4 = F8_CTX // 16
    N4 = F8_S * nb4
    k, v = pools(N4, torch.bfloat16)
    ks = float(k.float().abs().max()) / 448
    vs = float(v.float().abs().max()) / 448
    k8 = torch.empty(k.shape, dtype=torch.uint8, device="cuda")
    v8 = torch.empty_like(k8)
    tla.convert_fp8(k8, k, 1.0 / ks)
    tla.convert_fp8(v8, v, 1.0 / vs)
    torch.cuda.synchronize()
    del k, v
    tab4 = torch.randperm(N4, generator=g, device="cuda").to(torch.int32).view(F8_S, nb4).cpu().numpy()
    q4 = _host_u16(torch.randn(F8_S, H, D, generator=g, device="cuda").to(torch.bfloat16))
    k8h, v8h = k8.cpu().numpy(), v8.cpu().numpy()
    del k8, v8
    lens4 = np.full(F8_S, F8_CTX, np.int32)
    n4 = 2
    f4 = lambda th, n: (lambda: orc.paged_attention_f32(q4[:n], orc.BF16, k8h, v8h, orc.FP8, tab4[:n], lens4[:n],
                                                        NKV, sc, orc.GROUPED, threads=th, k_scale=ks, v_scale=vs))
    b4 = lambda n: n * F8_CTX * NKV * D * 2 + n * H * D * 2 * 2 + n * (nb4 * 4 + 4)
    entry("fp8_b16_ctx32768", "FP8 E4M3 KV (per-tensor scales), batch 16, ctx 32768, 32/8 heads, bf16 q",
          b4(F8_S), b4(n4), n4, F8_S, f4(ncore, F8_S), f4(1, n4))
    del k8h, v8h

    head = out["bf16_b64_ctx4096"]
    return {
        "value": head["all_cores"]["gbs"], "unit": "GB/s", "tok_s": head["all_cores"]["tok_s"], "cores": ncore,
        "kind": "port",
        "sample": f"the headline workload at full size (batch 64, ctx 4096, bf16): the oracle's fp32 decode on "
                  f"{ncore} threads, median of {head['all_cores']['runs']} runs; one thread over "
                  f"{head['single_thread']['sequences']} of the 64 sequences. Per workload: 'configs'",
        "single_thread": {"value": head["single_thread"]["gbs"], "unit": "GB/s",
                          "tok_s": head["single_thread"]["tok_s"]},
        "configs": out,
        "nproc": info["nproc"], "affinity_cpus": info["affinity"], "cpu_model": info["model"],
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "bench.py measures one GPU: --gpus must be 1 (the multi-GPU plan is design only)"}))
        sys.exit(2)
    if args.block_size != 16 and (args.only not in ("bf16", "fp16", "fp8") or (args.only == "fp8" and args.block_size < 16)):
        print(json.dumps({"error": "--block-size other than 16 applies to --only bf16, fp16 (8-256) or fp8 (16-256)"}))
        sys.exit(2)
    global BS
    BS = args.block_size

    import torch

    torch.cuda.set_device(0)
    for name in ("k0", "v0", "k1", "v1"):             # the pool arena first (pool_buffer)
        POOL_ARENA[name] = torch.empty(arena_bytes(), dtype=torch.uint8, device="cuda")
    global USE_GRAPH
    USE_GRAPH = not args.no_graph
    if args.copy_calibration:
        n = 1 << 30
        a = torch.empty(n, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_read": n, "bytes_written": n, "launches": 5}), flush=True)
        return
    res = {"metric": METRIC, "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "bf16", "data": "synthetic"}
    bf = fp = kv = None
    want = lambda *names: args.only == "all" or args.only in names
    if want("bf16", "v2"):
        bf = bench_decode(args, "bf16", name="bf16")
    if want("fp16", "kivi"):
        fp = bench_decode(args, "fp16", name="fp16")
    if want("kivi"):
        kv = bench_kivi(args, name="kivi")
    kvm = bench_kivi(args, mixed=True, name="kivi_mixed") if want("kivi") else None
    # the same two workloads with each page written in eighths over the 8
    # steps before the one that completes it (tl_kivi_desc.build_ahead)
    kva = bench_kivi(args, name="kivi_build_ahead", build_ahead=True) if want("kivi") else None
    kvma = bench_kivi(args, mixed=True, name="kivi_mixed_build_ahead", build_ahead=True) if want("kivi") else None
    kv8 = bench_kivi(args, name="kivi_int8", bits=8) if want("kivi") else None
    kvr = bench_kivi(args, name="kivi_pre_rope", pre_rope=True) if want("kivi") else None
    # the reference's default KiviConfig (config_schema.h:124,128): bits 8,
    # keys held before RoPE
    kvd = bench_kivi(args, name="kivi_default_config", bits=8, pre_rope=True) if want("kivi") else None
    fpa = bench_decode(args, "fp16", append=True, name="fp16_append") if want("kivi") else None
    f8 = bench_fp8(args, name="fp8") if want("fp8") else None
    f8p = bench_fp8(args, 512, name="fp8_pt512") if want("fp8") else None
    c2b = {}
    if want("config2b"):
        lens2b = config2b_lens()
        for label, pt in (("auto", 0), ("single_pass", -1), ("split_k_512", 512)):
            c2b[label] = bench_decode(args, "bf16", lens=lens2b, partition_tokens=pt, name=f"config2b_{label}")
    v2a = bench_decode(args, "bf16", v2=True, name="v2") if want("v2") else None
    # the engine's call shape: one sequence per call, 32 layers each with a
    # pool of its own (672 MB in all, beyond the 256 MiB Infinity Cache)
    v2one = bench_decode(args, "f16", lens=[CTX], v2=True, name="v2_one_seq", layers=32) if want("v2") else None
    # the same with the engine's whole v2 scratch: allocated once for
    # ceil(n_ctx_train / 512) partitions, 16 for a model trained at 8192
    v2cap = (bench_decode(args, "f16", lens=[CTX], v2=True, name="v2_one_seq_cap16", layers=32, v2_capacity=16)
             if want("v2") else None)
    one = bench_decode(args, "f16", lens=[CTX], name="auto_one_seq", layers=32) if want("v2") else None
    pf = bench_prefill(args) if args.only in ("all", "prefill") else None
    cb = bench_copy_blocks(args) if args.only in ("all", "blocks") else None
    rp = bench_rope(args) if args.only in ("all", "rope") else None
    vq = bench_vq(args) if args.only in ("all", "vq") else None
    na = bench_norm_act(args) if args.only in ("all", "norm") else None
    head = bf or fp
    if head is not None:
        res["dtype"] = "bf16" if bf else "fp16"
        res["value"] = round(head["gbs"], 2)
        res["ms_per_step"] = round(head["ms_per_step"], 5)
        res["pct_hbm_peak"] = round(100 * head["gbs"] / HBM_PEAK_GBS, 2)
        res["tok_s"] = round(head["tok_s"], 1)
        res["tok_s_32_layers"] = round(head["tok_s"] / 32, 1)
        achieved = head["bytes"] / (head["launch_ms"] * 1e-3) / 1e9
        res["roofline"] = {
            "kernel": "mfma2_decode_kernel (paged decode, single pass)" if head["workspace_bytes"] == 0
                      else "mfma2_decode_kernel + lse_reduce_kernel (split-K)",
            "bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "bytes_per_launch": head["bytes"],
            "traffic": traffic_from_profile(),
        }
    elif kv is not None:
        res["value"] = round(kv["gbs"], 2)
        res["ms_per_step"] = round(kv["ms_per_step"], 5)
        res["dtype"] = "f16 x int4"
    else:
        res["value"] = None
        res["unit"] = "GB/s (decode benches not run)"
    res["config"] = {
        "workload": "paged-attention decode, Llama-3-8B shape, one layer, batch 64, ctx 4096",
        "batch": S, "q_heads": H, "kv_heads": NKV, "head_dim": D, "block_size": BS, "context": CTX,
        "kv_dtype": res["dtype"], "pools_rotated": 2,
        "partition_tokens": args.partition_tokens or "auto",
    }
    res["timing"] = (f"ms_per_step = median over R replays of a HIP graph of --steps steps (R >= {MIN_REPLAYS}, "
                     f">= {MIN_TIMED_STEPS} timed steps), after untimed replays to sustained clocks")
    res["spread_ms_per_step"] = {k: {"min": round(v[0], 5), "max": round(v[1], 5), "replays": v[2], "steps": v[3]}
                                 for k, v in SPREAD.items()}
    if fp is not None:
        res["fp16"] = {"gbs": round(fp["gbs"], 2), "ms_per_step": round(fp["ms_per_step"], 5),
                       "tok_s": round(fp["tok_s"], 1),
                       "pct_hbm_peak": round(100 * fp["gbs"] / HBM_PEAK_GBS, 2)}
    if c2b:
        res["config2b_variable_lengths"] = {
            "workload": "bf16 decode, batch 64, lengths uniform in [512, 8192] (seed 0x7E5E0002), 32/8 heads, d 128, "
                        f"bs 16; mean length {sum(config2b_lens()) / S:.0f}",
            **{label: {"gbs": round(r["gbs"], 2), "pct_hbm_peak": round(100 * r["gbs"] / HBM_PEAK_GBS, 2),
                       "ms_per_step": round(r["ms_per_step"], 5), "tok_s": round(r["tok_s"], 1),
                       "partitions": r["partitions"], "bytes_per_step": r["bytes"]}
               for label, r in c2b.items()}}
    if v2a is not None:
        res["paged_attention_v2_dropin"] = {
            "workload": "tl_paged_attention_v2 (the operator the engine calls past 32 blocks) at batch 64, ctx 4096, "
                        "bf16, with the engine's scratch sizes",
            "gbs": round(v2a["gbs"], 2), "pct_hbm_peak": round(100 * v2a["gbs"] / HBM_PEAK_GBS, 2),
            "ms_per_step": round(v2a["ms_per_step"], 5),
            "vs_library_plan": round(bf["ms_per_step"] / v2a["ms_per_step"], 4) if bf else None}
    if v2one is not None:
        res["paged_attention_v2_one_sequence"] = {
            "workload": "the engine's own call: one sequence, ctx 4096, 32/8 heads, d 128, f16, "
                        "tl_paged_attention_v2 on the engine's scratch against tl_paged_attention_decode's plan; "
                        "32 layers with pools of their own (step i reads layer i % 32), "
                        f"{v2one['pool_bytes_all_layers'] / 1e6:.0f} MB in all, beyond the 256 MiB Infinity Cache",
            "v2_us": round(v2one["ms_per_step"] * 1e3, 2), "v2_partitions": v2one["partitions"],
            "v2_partition_tokens": v2one["partition_tokens"], "v2_gbs": round(v2one["gbs"], 2),
            "library_plan_us": round(one["ms_per_step"] * 1e3, 2) if one else None,
            "library_plan_partitions": one["partitions"] if one else None,
            "library_plan_gbs": round(one["gbs"], 2) if one else None}
        if v2cap is not None:
            res["paged_attention_v2_one_sequence"]["v2_engine_allocation"] = {
                "workload": "tl_paged_attention_v2_capacity with the scratch the engine allocates once for a "
                            "model trained at 8192 tokens (16 partitions, cuda_engine.cpp:273-285)",
                "us": round(v2cap["ms_per_step"] * 1e3, 2), "partitions": v2cap["partitions"],
                "partition_tokens": v2cap["partition_tokens"], "gbs": round(v2cap["gbs"], 2)}
    if kv is not None:
        res["kivi_int4"] = {"gbs": round(kv["gbs"], 2), "ms_per_step": round(kv["ms_per_step"], 5),
                            "tok_s": round(kv["tok_s"], 1),
                            "pct_hbm_peak": round(100 * kv["gbs"] / HBM_PEAK_GBS, 2),
                            "bytes_per_step": int(kv["bytes_per_step"]),
                            "steps": kv["steps"],
                            "includes": "append of 1 token/seq with quantise-on-append + decode, "
                                        "fp16 window through its whole 128..159-token cycle"}
        if fp is not None:
            res["kivi_int4"]["speedup_vs_fp16_tok_s"] = round(kv["tok_s"] / fp["tok_s"], 3)
        if fpa is not None:
            # like for like: the fp16 step with its append (reshape_and_cache,
            # then decode), as the KIVI step holds its own
            res["fp16_with_append"] = {"ms_per_step": round(fpa["ms_per_step"], 5),
                                       "tok_s": round(fpa["tok_s"], 1)}
            res["kivi_int4"]["speedup_vs_fp16_step_with_append"] = round(kv["tok_s"] / fpa["tok_s"], 3)
    if kvm is not None:
        res["kivi_int4_mixed_lengths"] = {
            "workload": "as kivi_int4, sequence s starting at 4096 + s mod 32 tokens: two sequences complete a page "
                        "at every step",
            "gbs": round(kvm["gbs"], 2), "ms_per_step": round(kvm["ms_per_step"], 5), "tok_s": round(kvm["tok_s"], 1),
            "pct_hbm_peak": round(100 * kvm["gbs"] / HBM_PEAK_GBS, 2), "bytes_per_step": int(kvm["bytes_per_step"])}
        if fp is not None:
            res["kivi_int4_mixed_lengths"]["speedup_vs_fp16_tok_s"] = round(kvm["tok_s"] / fp["tok_s"], 3)
    for key, r_ in (("kivi_int4", kva), ("kivi_int4_mixed_lengths", kvma)):
        if r_ is not None and key in res:
            res[key]["build_ahead"] = {"ms_per_step": round(r_["ms_per_step"], 5), "tok_s": round(r_["tok_s"], 1),
                                       "gbs": round(r_["gbs"], 2)}
            if fp is not None:
                res[key]["build_ahead"]["speedup_vs_fp16_tok_s"] = round(r_["tok_s"] / fp["tok_s"], 3)
    if kv8 is not None:
        res["kivi_int8"] = {
            "workload": "as kivi_int4 with INT8 pages (9216 B per 32 tokens per kv head)",
            "gbs": round(kv8["gbs"], 2), "ms_per_step": round(kv8["ms_per_step"], 5), "tok_s": round(kv8["tok_s"], 1),
            "pct_hbm_peak": round(100 * kv8["gbs"] / HBM_PEAK_GBS, 2), "bytes_per_step": int(kv8["bytes_per_step"])}
        if fp is not None:
            res["kivi_int8"]["speedup_vs_fp16_tok_s"] = round(kv8["tok_s"] / fp["tok_s"], 3)
    if kvr is not None:
        res["kivi_int4_pre_rope_keys"] = {
            "workload": "as kivi_int4 with the keys held before RoPE (pages and pool unrotated), every key rotated "
                        "at its position inside attention (halves style, fp32 tables of 8192 positions)",
            "gbs": round(kvr["gbs"], 2), "ms_per_step": round(kvr["ms_per_step"], 5), "tok_s": round(kvr["tok_s"], 1),
            "pct_hbm_peak": round(100 * kvr["gbs"] / HBM_PEAK_GBS, 2), "bytes_per_step": int(kvr["bytes_per_step"]),
            "rope_table_bytes_not_counted": True}
        if kv is not None:
            res["kivi_int4_pre_rope_keys"]["step_time_vs_rotated_keys"] = round(kvr["ms_per_step"] / kv["ms_per_step"], 3)
        if fp is not None:
            res["kivi_int4_pre_rope_keys"]["speedup_vs_fp16_tok_s"] = round(kvr["tok_s"] / fp["tok_s"], 3)
    if kvd is not None:
        res["kivi_default_config"] = {
            "workload": "the reference's default KiviConfig (bits 8, pre_rope_keys true; config_schema.h:124,128): "
                        "INT8 pages, keys held before RoPE and rotated at their positions inside attention, "
                        "batch 64, ctx 4096, one appended token per step",
            "gbs": round(kvd["gbs"], 2), "ms_per_step": round(kvd["ms_per_step"], 5), "tok_s": round(kvd["tok_s"], 1),
            "pct_hbm_peak": round(100 * kvd["gbs"] / HBM_PEAK_GBS, 2), "bytes_per_step": int(kvd["bytes_per_step"]),
            "rope_table_bytes_not_counted": True}
        if fp is not None:
            res["kivi_default_config"]["speedup_vs_fp16_tok_s"] = round(kvd["tok_s"] / fp["tok_s"], 3)
    if f8 is not None:
        res["fp8_e4m3_long_context"] = {
            "workload": "decode, batch 16, ctx 32768, 32 q / 8 kv heads, d 128, FP8 E4M3 KV with per-tensor "
                        f"scales, bf16 q, split-K {f8['partitions']} x {F8_CTX // f8['partitions']} tokens "
                        "(library plan) + LSE reduce",
            "gbs": round(f8["gbs"], 2), "pct_hbm_peak": round(100 * f8["gbs"] / HBM_PEAK_GBS, 2),
            "ms_per_step": round(f8["ms_per_step"], 5), "tok_s": round(f8["tok_s"], 1),
            "bytes_per_step": f8["bytes"], "split_k_partial_bytes_not_counted": f8["partial_bytes"]}
    if f8p is not None:
        res["fp8_e4m3_long_context_512_token_partitions"] = {
            "workload": "as fp8_e4m3_long_context, split-K into 64 partitions of 512 tokens (the workload's stated "
                        "partitioning) + LSE reduce",
            "gbs": round(f8p["gbs"], 2), "pct_hbm_peak": round(100 * f8p["gbs"] / HBM_PEAK_GBS, 2),
            "ms_per_step": round(f8p["ms_per_step"], 5), "tok_s": round(f8p["tok_s"], 1),
            "partitions": f8p["partitions"], "split_k_partial_bytes_not_counted": f8p["partial_bytes"]}
    if pf is not None:
        res["prefill"] = {
            "workload": "chunked prefill, 64 q / 8 kv heads, d 128, bf16: 8 prompts x 2048 tokens as 4 "
                        "causal 512-token chunk launches, each with 32 decode rows at ctx 2048",
            "tflops": round(pf["tflops"], 2), "pct_mfma_peak_bf16": round(100 * pf["tflops"] / 2500.0, 2),
            "ms_per_4_launches": round(pf["ms_per_step"], 5), "ms_per_launch": round(pf["ms_per_launch"], 5),
            "flops_per_4_launches": pf["flops"]}
    if cb is not None:
        res["copy_blocks"] = {
            "workload": f"copy_blocks, {CB_PAIRS} pairs of {NKV} x {D} x {BS} fp16 blocks (K and V pools of "
                        f"{CB_BLOCKS} blocks)",
            "gbs": round(cb["gbs"], 2), "pct_hbm_peak": round(100 * cb["gbs"] / HBM_PEAK_GBS, 2),
            "us_per_call": round(cb["ms"] * 1e3, 2), "bytes_per_call": cb["bytes"]}
    if rp is not None:
        res["rope_reshape_and_cache"] = {
            "workload": f"decode-step append, batch {S}: RoPE on q [{S}, {H}, {D}] and k, k and v into the bf16 "
                        "pools, one launch",
            "us_per_call": round(rp["us"], 2), "bytes_per_call": rp["bytes"],
            "gbs": round(rp["bytes"] / (rp["us"] * 1e-6) / 1e9, 2),
            "bf16_decode_us": round(rp["us_decode"], 2),
            "append_then_decode_us": round(rp["us_append_then_decode"], 2)}
    if vq is not None:
        res["vq_encode"] = {
            "workload": f"VQ encode, {VQ_N} fp16 vectors of d {D} against {VQ_K} entries (exact fp32 distances)",
            "us_per_call": round(vq["ms"] * 1e3, 2), "tflops_fp32": round(vq["tflops"], 2),
            "pct_fp32_vector_peak": round(100 * vq["tflops"] / 157.3, 2), "flops_per_call": vq["flops"]}
    if na is not None:
        res["norm_act"] = {
            "workload": f"bf16, {NA_ROWS} rows: fused_add_rms_norm [{NA_ROWS}, {NA_HID}], silu_and_mul "
                        f"[{NA_ROWS}, {NA_FFN}]",
            "fused_add_rms_norm_us": round(na["norm_us"], 2),
            "fused_add_rms_norm_gbs": round(na["norm_bytes"] / (na["norm_us"] * 1e-6) / 1e9, 2),
            "silu_and_mul_us": round(na["act_us"], 2),
            "silu_and_mul_gbs": round(na["act_bytes"] / (na["act_us"] * 1e-6) / 1e9, 2)}
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
