"""Parity of the FP8 E4M3 matrix-core decode (head_size 128, block_size 16)
against the oracle on the dequantised pools.

Tolerance: max-abs 1e-2 plus half an output ulp (as for every FP8 test).
The kernel widens codes to f16 exactly, so the remaining differences are
f16 weights and fp32 accumulation order."""
import math

import numpy as np
import pytest
import torch

import inputs
import oracle_lib as orc
import tl_attn as tla
from gpu_util import assert_close, dev, host_f64

pytestmark = pytest.mark.gpu

ATOL_FP8 = 1e-2
NAN_CODE = np.uint8(0x7F)


def _case(seed, lens, H, n_kv, q_code=orc.BF16, holes=0, q_mag=1.0):
    base = inputs.make_paged_case(seed, len(lens), H, n_kv, 128, 16, lens, orc.F32, holes=holes)
    ks = float(np.abs(base.k_cache).max()) / 448.0
    vs = float(np.abs(base.v_cache).max()) / 448.0
    k8 = orc.f32_to_e4m3(base.k_cache, np.float32(1.0) / np.float32(ks))
    v8 = orc.f32_to_e4m3(base.v_cache, np.float32(1.0) / np.float32(vs))
    q = inputs.encode(orc.bits_to_f32(base.q, orc.F32) * np.float32(q_mag), q_code)
    return base, q, k8, v8, ks, vs


def _run(base, q, q_code, k8, v8, ks, vs, n_kv, gqa, pt):
    qd = dev(q, q_code)
    kd, vd = torch.from_numpy(k8).cuda(), torch.from_numpy(v8).cuda()
    bt, sl = dev(base.tables), dev(base.seq_lens)
    max_ctx = int(base.seq_lens.max())
    desc = tla.make_decode_desc(qd, kd, bt, n_kv, base.scale, kv_dtype=tla.FP8_E4M3, gqa_map=gqa,
                                partition_tokens=pt, k_scale=ks, v_scale=vs)
    ws = torch.empty(max(16, tla.workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
    out = torch.full_like(qd, float("nan"))
    tla.paged_attention_decode(desc, out, qd, kd, vd, bt, sl, max_ctx, ws)
    torch.cuda.synchronize()
    return out


def _ref(base, q, q_code, k8, v8, ks, vs, n_kv, gqa):
    return orc.paged_attention(q, q_code, k8, v8, orc.FP8, base.tables, base.seq_lens, n_kv, base.scale,
                               gqa, 0, ks, vs)


@pytest.mark.parametrize("H,n_kv", [(4, 4), (6, 2), (16, 2), (32, 2), (64, 2)])
@pytest.mark.parametrize("pt", [-1, 512])
def test_fp8_group_sizes(H, n_kv, pt):
    """MHA, group 3, 8, 16 (all 16 MFMA columns) and 32 (two head slices),
    both GQA maps."""
    lens = [1500, 64, 700]
    base, q, k8, v8, ks, vs = _case(51, lens, H, n_kv)
    for gqa in (tla.GQA_MODULO, tla.GQA_GROUPED):
        print(f"case fp8 H={H} n_kv={n_kv} pt={pt} gqa={gqa}", flush=True)
        out = _run(base, q, orc.BF16, k8, v8, ks, vs, n_kv, gqa, pt)
        assert_close(out, _ref(base, q, orc.BF16, k8, v8, ks, vs, n_kv, gqa), orc.BF16, ATOL_FP8, "fp8")


EDGE_LENS = [0, 1, 15, 16, 17, 63, 64, 65, 511, 512, 513, 1023, 1025, 2047]


@pytest.mark.parametrize("q_code", [orc.F16, orc.BF16])
@pytest.mark.parametrize("pt", [-1, 512])
def test_fp8_edge_lengths_holes_and_nan_slots(q_code, pt):
    """Lengths around the 16-token block, the 64-token wavefront step and the
    512-token partition, table holes, and NaN codes in the unused slots of
    every last block: none of them reach the output; an empty sequence
    gives zeros."""
    base, q, k8, v8, ks, vs = _case(52, EDGE_LENS, 8, 2, q_code=q_code, holes=5)
    for s, L in enumerate(EDGE_LENS):
        if L % 16:
            last = base.tables[s, (L - 1) // 16]
            if last >= 0:
                k8[last, :, :, L % 16:] = NAN_CODE
                v8[last, :, :, L % 16:] = NAN_CODE
    print(f"case fp8 edges q={q_code} pt={pt}", flush=True)
    out = _run(base, q, q_code, k8, v8, ks, vs, 2, tla.GQA_GROUPED, pt)
    assert_close(out, _ref(base, q, q_code, k8, v8, ks, vs, 2, tla.GQA_GROUPED), q_code, ATOL_FP8, "fp8")
    assert (host_f64(out[0]) == 0).all()


@pytest.mark.parametrize("q_mag", [3e4, 1e-5])
def test_fp8_bf16_q_magnitudes(q_mag):
    """bf16 q far outside [2^-14, 2^15) (where f16 would overflow or lose
    bits) is brought into range by a power of two per head; the scores are
    the same.  The softmax scale is divided by the magnitude so the weights
    stay comparable."""
    lens = [900, 300]
    base, q, k8, v8, ks, vs = _case(53, lens, 8, 2, q_mag=q_mag)
    base.scale = base.scale / q_mag
    print(f"case fp8 q_mag={q_mag}", flush=True)
    out = _run(base, q, orc.BF16, k8, v8, ks, vs, 2, tla.GQA_GROUPED, -1)
    assert_close(out, _ref(base, q, orc.BF16, k8, v8, ks, vs, 2, tla.GQA_GROUPED), orc.BF16, ATOL_FP8, "fp8")


def test_fp8_long_context_single_pass_equals_split_k_and_spot_checks():
    """Batch 16, ctx 32768, 32/8 heads, bf16 q, per-tensor scales, shuffled
    1.25x pool: single pass and 64 x 512 split-K agree, and two sequences
    match the oracle."""
    S, H, n_kv, D, BS, L = 16, 32, 8, 128, 16, 32768
    g = torch.Generator(device="cuda").manual_seed(inputs.SEEDS[0])
    nb = L // BS
    N = math.ceil(1.25 * S * nb)
    perm = torch.randperm(N, generator=g, device="cuda").to(torch.int32)
    tables = perm[: S * nb].view(S, nb).contiguous()
    kf = torch.randn(N, n_kv, D, BS, generator=g, device="cuda", dtype=torch.float16)
    vf = torch.randn(N, n_kv, D, BS, generator=g, device="cuda", dtype=torch.float16)
    ks = kf.abs().max().item() / 448.0
    vs = vf.abs().max().item() / 448.0
    k8 = (kf.float() / ks).to(torch.float8_e4m3fn).view(torch.uint8)
    v8 = (vf.float() / vs).to(torch.float8_e4m3fn).view(torch.uint8)
    del kf, vf
    q = torch.randn(S, H, D, generator=g, device="cuda").to(torch.bfloat16)
    sl = torch.full((S,), L, dtype=torch.int32, device="cuda")
    scale = 1 / math.sqrt(D)
    outs = {}
    for pt in (-1, 512, 0):
        desc = tla.make_decode_desc(q, k8, tables, n_kv, scale, kv_dtype=tla.FP8_E4M3, partition_tokens=pt,
                                    k_scale=ks, v_scale=vs)
        ws = torch.empty(max(16, tla.workspace_bytes(desc, L)), dtype=torch.uint8, device="cuda")
        out = torch.empty_like(q)
        print(f"case fp8 long-context pt={pt}", flush=True)
        tla.paged_attention_decode(desc, out, q, k8, v8, tables, sl, L, ws)
        torch.cuda.synchronize()
        outs[pt] = out.float()
    for pt in (512, 0):
        assert (outs[pt] - outs[-1]).abs().max().item() <= 2 * ATOL_FP8
    tb = tables.cpu().numpy()
    for s in (0, 15):
        idx = torch.from_numpy(tb[s].astype(np.int64)).cuda()
        sub_k = k8[idx].contiguous().cpu().numpy()
        sub_v = v8[idx].contiguous().cpu().numpy()
        qs = q[s:s + 1].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
        ref = orc.paged_attention(qs, orc.BF16, sub_k, sub_v, orc.FP8, np.arange(nb, dtype=np.int32)[None],
                                  np.array([L], np.int32), n_kv, scale, orc.GROUPED, 0, ks, vs)
        assert_close(outs[512][s:s + 1].to(torch.bfloat16), ref, orc.BF16, ATOL_FP8, f"seq {s}")


def test_fp8_graph_replay_matches_eager():
    """The split-K FP8 decode captured in a HIP graph and replayed with eager
    work between: bit-equal to the eager launch (no data-dependent
    scheduling)."""
    lens = [4096, 1000, 17, 1, 0, 2047]
    base, q, k8, v8, ks, vs = _case(54, lens, 32, 8)
    qd = dev(q, orc.BF16)
    kd, vd = torch.from_numpy(k8).cuda(), torch.from_numpy(v8).cuda()
    bt, sl = dev(base.tables), dev(base.seq_lens)
    desc = tla.make_decode_desc(qd, kd, bt, 8, base.scale, kv_dtype=tla.FP8_E4M3, partition_tokens=512,
                                k_scale=ks, v_scale=vs)
    ws = torch.empty(max(16, tla.workspace_bytes(desc, 4096)), dtype=torch.uint8, device="cuda")
    out = torch.zeros_like(qd)
    print("case fp8 graph replay", flush=True)
    tla.paged_attention_decode(desc, out, qd, kd, vd, bt, sl, 4096, ws)
    torch.cuda.synchronize()
    eager = out.clone()
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    with torch.cuda.graph(graph, stream=cap):
        tla.paged_attention_decode(desc, out, qd, kd, vd, bt, sl, 4096, ws, cap)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        tla.paged_attention_decode(desc, out, qd, kd, vd, bt, sl, 4096, ws)
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


RAGGED = [32768, 1, 0, 511, 512, 513, 16385, 4097, 32767, 8191, 1025, 3, 12345, 30000, 64, 700]


@pytest.mark.parametrize("kv", ["fp8", "bf16"])
@pytest.mark.parametrize("H", [32, 64, 128])
def test_whole_partitions_per_wavefront_ragged_lengths(kv, H):
    """Split-K at 512-token partitions with at least 4096 partitions runs
    whole partitions per wavefront (4 per wavefront here), the finished ones
    kept in LDS until the wavefront's last loads (groups 4 and 8) or written
    at once (group 16, whose slots would not fit): ragged lengths, empty and
    one-token sequences, partition edges, against the single-pass kernel
    (itself checked against the oracle by the tests above)."""
    S, n_kv, D, BS = len(RAGGED), 8, 128, 16
    g = torch.Generator(device="cuda").manual_seed(inputs.SEEDS[1] + H)
    nbs = [(L + BS - 1) // BS for L in RAGGED]
    mb = max(nbs)
    N = sum(nbs) + 5
    perm = torch.randperm(N, generator=g, device="cuda").to(torch.int32)
    tables = torch.full((S, mb), -1, dtype=torch.int32, device="cuda")
    off = 0
    for s, nb in enumerate(nbs):
        tables[s, :nb] = perm[off:off + nb]
        off += nb
    q = torch.randn(S, H, D, generator=g, device="cuda").to(torch.bfloat16)
    if kv == "fp8":
        kf = torch.randn(N, n_kv, D, BS, generator=g, device="cuda", dtype=torch.float16)
        vf = torch.randn(N, n_kv, D, BS, generator=g, device="cuda", dtype=torch.float16)
        ks, vs = kf.abs().max().item() / 448.0, vf.abs().max().item() / 448.0
        k = (kf.float() / ks).to(torch.float8_e4m3fn).view(torch.uint8)
        v = (vf.float() / vs).to(torch.float8_e4m3fn).view(torch.uint8)
        del kf, vf
        extra = dict(kv_dtype=tla.FP8_E4M3, k_scale=ks, v_scale=vs)
        tol = ATOL_FP8
    else:
        k = torch.randn(N, n_kv, D, BS, generator=g, device="cuda").to(torch.bfloat16)
        v = torch.randn(N, n_kv, D, BS, generator=g, device="cuda").to(torch.bfloat16)
        extra = {}
        tol = 2e-3
    sl = torch.tensor(RAGGED, dtype=torch.int32, device="cuda")
    L = max(RAGGED)
    scale = 1 / math.sqrt(D)
    outs = {}
    for pt in (-1, 512):
        desc = tla.make_decode_desc(q, k, tables, n_kv, scale, partition_tokens=pt, **extra)
        ws = torch.empty(max(16, tla.workspace_bytes(desc, L)), dtype=torch.uint8, device="cuda")
        out = torch.full_like(q, float("nan"))
        print(f"case whole partitions kv={kv} H={H} pt={pt}", flush=True)
        tla.paged_attention_decode(desc, out, q, k, v, tables, sl, L, ws)
        torch.cuda.synchronize()
        outs[pt] = out.float()
    empty = torch.tensor(RAGGED, device="cuda") == 0
    assert (outs[512][empty] == 0).all() and (outs[-1][empty] == 0).all()
    assert torch.isfinite(outs[512]).all()
    assert (outs[512] - outs[-1]).abs().max().item() <= 2 * tol
