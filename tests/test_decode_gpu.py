"""Parity of the gfx950 paged-attention decode against the oracle.

Tolerance: max-abs 2e-3 for fp16 / bf16 / fp32 KV and 1e-2 for FP8 KV
(against attention on the dequantised pool), each plus half an ulp of the
output dtype at the exact value (the rounding of the stored result)."""
import math

import numpy as np
import pytest
import torch

import inputs
import oracle_lib as orc
import tl_attn as tla
from gpu_util import assert_close, dev, host_f64

pytestmark = pytest.mark.gpu

ATOL = 2e-3
ATOL_FP8 = 1e-2


def _gpu_case(case):
    return (dev(case.q, case.code), dev(case.k_cache, case.code), dev(case.v_cache, case.code),
            dev(case.tables), dev(case.seq_lens))


def _ref(case, gqa):
    return orc.paged_attention(case.q, case.code, case.k_cache, case.v_cache, case.code,
                               case.tables, case.seq_lens, case.num_kv_heads, case.scale, gqa)


def run_v1(case, gqa):
    q, k, v, bt, sl = _gpu_case(case)
    out = torch.full_like(q, float("nan"))
    tla.paged_attention_v1(out, q, k, v, bt, sl, case.num_kv_heads, case.scale, q.shape[2],
                           k.shape[3], gqa_map=gqa)
    torch.cuda.synchronize()
    return out


def run_v2(case, gqa):
    q, k, v, bt, sl = _gpu_case(case)
    S, H, D = q.shape
    max_ctx = int(case.seq_lens.max()) if len(case.seq_lens) else 0
    P = tla.v2_num_partitions(max_ctx, k.shape[3])
    es = torch.zeros(S, H, P, dtype=torch.float32, device="cuda")
    ml = torch.zeros(S, H, P, dtype=torch.float32, device="cuda")
    tmp = torch.zeros(S, H, P, D, dtype=q.dtype, device="cuda")
    out = torch.full_like(q, float("nan"))
    tla.paged_attention_v2(out, es, ml, tmp, q, k, v, bt, sl, case.num_kv_heads, case.scale, D,
                           k.shape[3], max_ctx, gqa_map=gqa)
    torch.cuda.synchronize()
    return out


def run_decode(case, gqa, partition_tokens=0):
    q, k, v, bt, sl = _gpu_case(case)
    max_ctx = int(case.seq_lens.max()) if len(case.seq_lens) else 0
    desc = tla.make_decode_desc(q, k, bt, case.num_kv_heads, case.scale, gqa_map=gqa,
                                partition_tokens=partition_tokens)
    nbytes = tla.workspace_bytes(desc, max_ctx)
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device="cuda")
    out = torch.full_like(q, float("nan"))
    tla.paged_attention_decode(desc, out, q, k, v, bt, sl, max_ctx, ws)
    torch.cuda.synchronize()
    return out


RUNNERS = {
    "v1": run_v1,
    "v2": run_v2,
    "auto": run_decode,
    "pt512": lambda c, g: run_decode(c, g, 512),
    "pt1024": lambda c, g: run_decode(c, g, 1024),
}


@pytest.mark.parametrize("gqa", [tla.GQA_MODULO, tla.GQA_GROUPED])
@pytest.mark.parametrize("runner", ["v1", "v2", "auto", "pt512"])
def test_fp16_batch4_reference_workload(runner, gqa):
    """Batch 4, 32/8 heads, d 128, bs 16, L ~ U[128, 1024], 512-block pool."""
    lens = inputs.uniform_lens(inputs.SEEDS[0], 4, 128, 1024)
    case = inputs.make_paged_case(inputs.SEEDS[0], 4, 32, 8, 128, 16, lens, orc.F16,
                                  num_blocks=512, max_blocks=64)
    print(f"case fp16 S=4 lens={list(lens)} runner={runner} gqa={gqa}", flush=True)
    assert_close(RUNNERS[runner](case, gqa), _ref(case, gqa), orc.F16, ATOL, runner)


@pytest.mark.parametrize("runner", ["v1", "v2", "auto", "pt512", "pt1024"])
def test_bf16_llama_shape_variable_lengths(runner):
    """32/8 heads, d 128, bs 16, L ~ U[512, 8192] (6 sequences)."""
    lens = inputs.uniform_lens(inputs.SEEDS[1], 6, 512, 8192)
    case = inputs.make_paged_case(inputs.SEEDS[1], 6, 32, 8, 128, 16, lens, orc.BF16)
    print(f"case bf16 lens={list(lens)} runner={runner}", flush=True)
    assert_close(RUNNERS[runner](case, tla.GQA_GROUPED), _ref(case, tla.GQA_GROUPED), orc.BF16,
                 ATOL, runner)


EDGE_LENS = [0, 1, 15, 16, 17, 511, 512, 513, 1023, 1025, 2047]


@pytest.mark.parametrize("runner", ["v1", "v2", "pt512"])
def test_edge_lengths_and_holes(runner):
    case = inputs.make_paged_case(31, len(EDGE_LENS), 8, 2, 128, 16, EDGE_LENS, orc.F16, holes=4)
    print(f"case edges runner={runner}", flush=True)
    out = RUNNERS[runner](case, tla.GQA_GROUPED)
    assert_close(out, _ref(case, tla.GQA_GROUPED), orc.F16, ATOL, runner)
    assert (host_f64(out[0]) == 0).all()                     # empty sequence -> zeros


@pytest.mark.parametrize("H,n_kv", [(8, 2), (4, 4)])
@pytest.mark.parametrize("code", [orc.F16, orc.BF16])
@pytest.mark.parametrize("runner", ["v1", "pt512"])
def test_unused_slots_holding_nan_are_ignored(code, runner, H, n_kv):
    """Slots past seq_len in a sequence's last block (and blocks past it) may
    hold anything, NaN included; they must not reach the output."""
    lens = [33, 500, 1031]
    case = inputs.make_paged_case(34, 3, H, n_kv, 128, 16, lens, code)
    nan = np.uint16(0x7E00 if code == orc.F16 else 0x7FC0)
    for s, L in enumerate(lens):
        last = case.tables[s, (L - 1) // 16]
        case.k_cache[last, :, :, L % 16 or 16:] = nan
        case.v_cache[last, :, :, L % 16 or 16:] = nan
    print(f"case nan-slots code={code} runner={runner}", flush=True)
    assert_close(RUNNERS[runner](case, tla.GQA_GROUPED), _ref(case, tla.GQA_GROUPED), code, ATOL,
                 runner)


@pytest.mark.parametrize("H,n_kv", [(4, 4), (6, 2), (16, 2), (8, 1)])
@pytest.mark.parametrize("runner", ["v1", "pt512"])
def test_gqa_group_sizes(H, n_kv, runner):
    """MHA, group 3 (padded), group 8 (two head slices), MQA."""
    lens = inputs.uniform_lens(32, 3, 1, 1500)
    case = inputs.make_paged_case(32, 3, H, n_kv, 128, 16, lens, orc.BF16)
    for gqa in (tla.GQA_MODULO, tla.GQA_GROUPED):
        print(f"case H={H} n_kv={n_kv} gqa={gqa} runner={runner}", flush=True)
        assert_close(RUNNERS[runner](case, gqa), _ref(case, gqa), orc.BF16, ATOL, runner)


@pytest.mark.parametrize("D,BS,code", [(64, 16, orc.F16), (256, 16, orc.F16), (128, 32, orc.F16),
                                       (64, 16, orc.BF16), (128, 16, orc.F32)])
@pytest.mark.parametrize("runner", ["v1", "pt512"])
def test_head_and_block_sizes(D, BS, code, runner):
    lens = inputs.uniform_lens(33, 3, 1, 1300)
    case = inputs.make_paged_case(33, 3, 8, 2, D, BS, lens, code)
    print(f"case D={D} BS={BS} code={code} runner={runner}", flush=True)
    assert_close(RUNNERS[runner](case, tla.GQA_GROUPED), _ref(case, tla.GQA_GROUPED), code, ATOL,
                 runner)


def _fp8_case(seed, S, lens, H=32, n_kv=8, D=128, BS=16, q_code=orc.F16):
    base = inputs.make_paged_case(seed, S, H, n_kv, D, BS, lens, orc.F32)
    ks = float(np.abs(base.k_cache).max()) / 448.0
    vs = float(np.abs(base.v_cache).max()) / 448.0
    k8 = orc.f32_to_e4m3(base.k_cache, np.float32(1.0) / np.float32(ks))
    v8 = orc.f32_to_e4m3(base.v_cache, np.float32(1.0) / np.float32(vs))
    q = inputs.encode(orc.bits_to_f32(base.q, orc.F32), q_code)
    return base, q, k8, v8, ks, vs


@pytest.mark.parametrize("q_code", [orc.F16, orc.BF16])
@pytest.mark.parametrize("pt", [-1, 512, 0])
def test_fp8_kv_decode(q_code, pt):
    """E4M3 pools with per-tensor scales absmax/448; compared with attention
    on the dequantised pool."""
    lens = [4096, 700, 1]
    base, q, k8, v8, ks, vs = _fp8_case(41, 3, lens, q_code=q_code)
    ref = orc.paged_attention(q, q_code, k8, v8, orc.FP8, base.tables, base.seq_lens, 8,
                              base.scale, orc.GROUPED, 0, ks, vs)
    qd = dev(q, q_code)
    kd, vd = torch.from_numpy(k8).cuda(), torch.from_numpy(v8).cuda()
    bt, sl = dev(base.tables), dev(base.seq_lens)
    desc = tla.make_decode_desc(qd, kd, bt, 8, base.scale, kv_dtype=tla.FP8_E4M3,
                                gqa_map=tla.GQA_GROUPED, partition_tokens=pt, k_scale=ks,
                                v_scale=vs)
    ws = torch.empty(max(16, tla.workspace_bytes(desc, 4096)), dtype=torch.uint8, device="cuda")
    out = torch.full_like(qd, float("nan"))
    print(f"case fp8 q={q_code} pt={pt}", flush=True)
    tla.paged_attention_decode(desc, out, qd, kd, vd, bt, sl, 4096, ws)
    torch.cuda.synchronize()
    assert_close(out, ref, q_code, ATOL_FP8, "fp8")


def test_fp8_decode_of_every_code_is_exact():
    """A one-token sequence returns v exactly: covers the hardware E4M3
    decoder on all 256 codes (NaN codes give NaN)."""
    D, BS = 128, 16
    codes = np.arange(256, dtype=np.uint8)
    k8 = np.zeros((2, 1, D, BS), np.uint8)
    v8 = np.zeros((2, 1, D, BS), np.uint8)
    v8[0, 0, :, 0] = codes[:128]
    v8[1, 0, :, 0] = codes[128:]
    q = inputs.encode(np.ones((2, 1, D), np.float32), orc.F16)
    tables = np.array([[0], [1]], np.int32)
    lens = np.array([1, 1], np.int32)
    vs = 0.5
    qd = dev(q, orc.F16)
    kd, vd = torch.from_numpy(k8).cuda(), torch.from_numpy(v8).cuda()
    desc = tla.make_decode_desc(qd, kd, dev(tables), 1, 0.1, kv_dtype=tla.FP8_E4M3,
                                partition_tokens=-1, k_scale=1.0, v_scale=vs)
    out = torch.empty_like(qd)
    tla.paged_attention_decode(desc, out, qd, kd, vd, dev(tables), dev(lens), 1)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy().reshape(256)
    want = (orc.bits_to_f32(codes, orc.FP8) * np.float32(vs)).astype(np.float16).astype(np.float32)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok], want[ok])


def test_full_size_single_pass_equals_split_k_and_spot_checks():
    """Batch 64, ctx 4096, 32/8 heads, d 128, bf16, shuffled 1.25x pool:
    single pass and split-K agree, and 3 sequences match the oracle."""
    S, H, n_kv, D, BS, L = 64, 32, 8, 128, 16, 4096
    g = torch.Generator(device="cuda").manual_seed(inputs.SEEDS[1])
    nb = L // BS
    N = math.ceil(1.25 * S * nb)
    perm = torch.randperm(N, generator=g, device="cuda").to(torch.int32)
    tables = perm[: S * nb].view(S, nb).contiguous()
    k = torch.randn(N, n_kv, D, BS, generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn(N, n_kv, D, BS, generator=g, device="cuda").to(torch.bfloat16)
    q = torch.randn(S, H, D, generator=g, device="cuda").to(torch.bfloat16)
    sl = torch.full((S,), L, dtype=torch.int32, device="cuda")
    scale = 1 / math.sqrt(D)
    outs = {}
    for pt in (-1, 512, 1024, 0):
        desc = tla.make_decode_desc(q, k, tables, n_kv, scale, partition_tokens=pt)
        ws = torch.empty(max(16, tla.workspace_bytes(desc, L)), dtype=torch.uint8, device="cuda")
        out = torch.empty_like(q)
        print(f"case full-size pt={pt}", flush=True)
        tla.paged_attention_decode(desc, out, q, k, v, tables, sl, L, ws)
        torch.cuda.synchronize()
        outs[pt] = out.float()
    for pt in (512, 1024, 0):
        assert (outs[pt] - outs[-1]).abs().max().item() <= 2 * ATOL
    tb = tables.cpu().numpy()
    for s in (0, 31, 63):
        blocks = tb[s]
        sub_k = k[blocks.tolist()].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
        sub_v = v[blocks.tolist()].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
        qs = q[s:s + 1].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
        ref = orc.paged_attention(qs, orc.BF16, sub_k, sub_v, orc.BF16,
                                  np.arange(nb, dtype=np.int32)[None], np.array([L], np.int32),
                                  n_kv, scale, orc.GROUPED)
        assert_close(outs[-1][s:s + 1].to(torch.bfloat16), ref, orc.BF16, ATOL, f"seq {s}")


def _oracle_one_sequence(q, k, v, tables, s, L, n_kv, scale, code):
    """The oracle on sequence s alone: its blocks gathered into a small pool."""
    nb = (L + k.shape[3] - 1) // k.shape[3]
    blocks = tables[s, :nb].tolist()
    sub_k = k[blocks].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    sub_v = v[blocks].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    qs = q[s:s + 1].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    return orc.paged_attention(qs, code, sub_k, sub_v, code, np.arange(nb, dtype=np.int32)[None],
                               np.array([L], np.int32), n_kv, scale, orc.GROUPED)


def test_full_batch_variable_lengths_every_plan_against_oracle():
    """The variable-length workload at its full size: batch 64, lengths
    uniform in [512, 8192], 32/8 heads, d 128, bs 16, bf16, tables a shuffled
    1.25x pool.  The library's own plan (4 partitions of 2048 tokens at this
    batch), the reference's 512-token partitions and single pass all agree,
    and 16 sequences spread over the batch (every fourth, the longest and the
    shortest among them) match the oracle under each plan."""
    S, H, n_kv, D, BS = 64, 32, 8, 128, 16
    lens = inputs.uniform_lens(inputs.SEEDS[1], S, 512, 8192)
    nbs = (lens + BS - 1) // BS
    N = math.ceil(1.25 * int(nbs.sum()))
    g = torch.Generator(device="cuda").manual_seed(inputs.SEEDS[1] + 2)
    perm = torch.randperm(N, generator=g, device="cuda").to(torch.int32)
    M = int(nbs.max())
    tables = torch.full((S, M), -1, dtype=torch.int32, device="cuda")
    off = 0
    for s in range(S):
        tables[s, : nbs[s]] = perm[off: off + nbs[s]]
        off += int(nbs[s])
    k = torch.randn(N, n_kv, D, BS, generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn(N, n_kv, D, BS, generator=g, device="cuda").to(torch.bfloat16)
    q = torch.randn(S, H, D, generator=g, device="cuda").to(torch.bfloat16)
    sl = torch.tensor(lens, dtype=torch.int32, device="cuda")
    scale = 1 / math.sqrt(D)
    max_ctx = int(lens.max())
    outs = {}
    for pt in (0, 512, -1):
        desc = tla.make_decode_desc(q, k, tables, n_kv, scale, partition_tokens=pt)
        if pt == 0:
            assert tla.workspace_bytes(desc, max_ctx) == S * H * 4 * (D + 2) * 4   # 4 partitions
        ws = torch.empty(max(16, tla.workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
        out = torch.full_like(q, float("nan"))
        print(f"case full-batch variable lengths pt={pt}", flush=True)
        tla.paged_attention_decode(desc, out, q, k, v, tables, sl, max_ctx, ws)
        torch.cuda.synchronize()
        outs[pt] = out
    for pt in (512, -1):
        assert (outs[pt].float() - outs[0].float()).abs().max().item() <= 2 * ATOL
    picks = sorted(set(range(0, S, 4)) | {int(np.argmax(lens)), int(np.argmin(lens))})
    tb = tables.cpu().numpy()
    for s in picks:
        ref = _oracle_one_sequence(q, k, v, tb, s, int(lens[s]), n_kv, scale, orc.BF16)
        for pt, out in outs.items():
            assert_close(out[s:s + 1], ref, orc.BF16, ATOL, f"seq {s} L={lens[s]} pt={pt}")


@pytest.mark.parametrize("pt", [-1, 512])
def test_decode_graph_replay_matches_eager(pt):
    """Decode (single pass and split-K + reduce) captured in a HIP graph and
    replayed three times with eager work between: every replay is bit-equal
    to the eager launch."""
    case = inputs.make_paged_case(inputs.SEEDS[2], 8, 32, 8, 128, 16,
                                  [4096, 1000, 17, 1, 0, 2047, 3000, 511], orc.BF16)
    q, k, v, bt, sl = _gpu_case(case)
    max_ctx = int(case.seq_lens.max())
    desc = tla.make_decode_desc(q, k, bt, case.num_kv_heads, case.scale, partition_tokens=pt)
    ws = torch.empty(max(16, tla.workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
    out = torch.zeros_like(q)
    print(f"case decode graph replay pt={pt}", flush=True)
    tla.paged_attention_decode(desc, out, q, k, v, bt, sl, max_ctx, ws)
    torch.cuda.synchronize()
    eager = out.clone()
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    with torch.cuda.graph(graph, stream=cap):
        tla.paged_attention_decode(desc, out, q, k, v, bt, sl, max_ctx, ws, cap)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        tla.paged_attention_decode(desc, out, q, k, v, bt, sl, max_ctx, ws)
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


@pytest.mark.parametrize("lens,code,kv", [
    ([4096], orc.F16, None), ([4097], orc.BF16, None), ([3000, 1200], orc.F16, None), ([1024], orc.F16, None),
    ([700, 33], orc.BF16, None), ([8000], orc.BF16, "fp8"), ([2500], orc.F16, "fp8"),
])
def test_small_batch_plan_against_oracle(lens, code, kv):
    """A batch too small to fill the GPU in 512-token partitions (the
    engine's one-sequence call): the plan takes partitions down to one
    iteration per wavefront (128 tokens of 2-byte KV, 256 of FP8) and merges
    up to 32 of them.  Against the oracle, with holes; the same case through
    the v2 operator with the engine's scratch (f16 partial outputs for f16)."""
    S = len(lens)
    if kv is None:
        case = inputs.make_paged_case(170 + S, S, 32, 8, 128, 16, lens, code, holes=1)
        q, k, v, bt, sl = _gpu_case(case)
        desc = tla.make_decode_desc(q, k, bt, 8, case.scale, gqa_map=tla.GQA_GROUPED)
        ref = _ref(case, tla.GQA_GROUPED)
        atol = ATOL
    else:
        case = inputs.make_paged_case(180 + S, S, 32, 8, 128, 16, lens, orc.F32, holes=1)
        ks = float(np.abs(case.k_cache).max()) / 448
        vs = float(np.abs(case.v_cache).max()) / 448
        k8, v8 = orc.f32_to_e4m3(case.k_cache, 1 / ks), orc.f32_to_e4m3(case.v_cache, 1 / vs)
        qn = inputs.encode(orc.bits_to_f32(case.q, orc.F32), code)
        ref = orc.paged_attention(qn, code, k8, v8, orc.FP8, case.tables, case.seq_lens, 8, case.scale, orc.GROUPED,
                                  0, ks, vs)
        q, k, v, bt, sl = dev(qn, code), dev(k8), dev(v8), dev(case.tables), dev(case.seq_lens)
        desc = tla.make_decode_desc(q, k, bt, 8, case.scale, gqa_map=tla.GQA_GROUPED, kv_dtype=tla.FP8_E4M3,
                                    k_scale=ks, v_scale=vs)
        atol = ATOL_FP8
    max_ctx = int(max(lens))
    nbytes = tla.workspace_bytes(desc, max_ctx)
    P = nbytes // (S * 32 * (128 + 2) * 4)
    assert P > -(-max_ctx // 512), P                   # finer than 512-token partitions
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device="cuda")
    out = torch.full_like(q, float("nan"))
    print(f"case small-batch plan lens={lens} code={code} kv={kv} P={P}", flush=True)
    tla.paged_attention_decode(desc, out, q, k, v, bt, sl, max_ctx, ws)
    torch.cuda.synchronize()
    assert_close(out, ref, code, atol, f"small batch {lens}")
    if kv is None:
        o2 = run_v2(case, tla.GQA_GROUPED)
        assert_close(o2, ref, code, ATOL, f"v2 small batch {lens}")
