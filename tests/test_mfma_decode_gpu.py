"""Parity of the 2-byte matrix-core decode (head_size 128, block_size 16:
one workgroup serves up to 16 q heads from one KV read) against the oracle,
here for GQA groups above 4, which a 4-head wavefront would read twice or
more (the other decode tests cover groups 1-4 on the same kernels).

Tolerance: max-abs 2e-3 plus half an output ulp, as for the other 2-byte
decode paths."""
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


def _run(case, gqa, pt):
    q, k, v = dev(case.q, case.code), dev(case.k_cache, case.code), dev(case.v_cache, case.code)
    bt, sl = dev(case.tables), dev(case.seq_lens)
    max_ctx = int(case.seq_lens.max())
    desc = tla.make_decode_desc(q, k, bt, case.num_kv_heads, case.scale, gqa_map=gqa, partition_tokens=pt)
    ws = torch.empty(max(16, tla.workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
    out = torch.full_like(q, float("nan"))
    tla.paged_attention_decode(desc, out, q, k, v, bt, sl, max_ctx, ws)
    torch.cuda.synchronize()
    return out


def _ref(case, gqa):
    return orc.paged_attention(case.q, case.code, case.k_cache, case.v_cache, case.code, case.tables,
                               case.seq_lens, case.num_kv_heads, case.scale, gqa)


@pytest.mark.parametrize("H,n_kv", [(12, 2), (16, 2), (32, 2), (64, 2), (64, 8)])
@pytest.mark.parametrize("code", [orc.F16, orc.BF16])
@pytest.mark.parametrize("pt", [-1, 512])
def test_mfma_decode_group_sizes(H, n_kv, code, pt):
    """Groups 6, 8, 16, 32 (two head slices) and the 64/8 shape, both GQA maps."""
    lens = inputs.uniform_lens(61, 3, 1, 1500)
    case = inputs.make_paged_case(61, 3, H, n_kv, 128, 16, lens, code)
    for gqa in (tla.GQA_MODULO, tla.GQA_GROUPED):
        print(f"case mfma2 H={H} n_kv={n_kv} code={code} pt={pt} gqa={gqa}", flush=True)
        assert_close(_run(case, gqa, pt), _ref(case, gqa), code, ATOL, "mfma2")


EDGE_LENS = [0, 1, 15, 16, 17, 31, 32, 33, 511, 512, 513, 1023, 1025, 2047]


@pytest.mark.parametrize("code", [orc.F16, orc.BF16])
@pytest.mark.parametrize("pt", [-1, 512])
def test_mfma_decode_edges_holes_and_nan_slots(code, pt):
    """Lengths around the block, the 32-token step and the partition, table
    holes, and NaN in every unused slot of a last block: none reach the
    output; an empty sequence gives zeros."""
    case = inputs.make_paged_case(62, len(EDGE_LENS), 16, 2, 128, 16, EDGE_LENS, code, holes=5)
    nan = np.uint16(0x7E00 if code == orc.F16 else 0x7FC0)
    for s, L in enumerate(EDGE_LENS):
        if L % 16:
            last = case.tables[s, (L - 1) // 16]
            if last >= 0:
                case.k_cache[last, :, :, L % 16:] = nan
                case.v_cache[last, :, :, L % 16:] = nan
    print(f"case mfma2 edges code={code} pt={pt}", flush=True)
    out = _run(case, tla.GQA_GROUPED, pt)
    assert_close(out, _ref(case, tla.GQA_GROUPED), code, ATOL, "mfma2")
    assert (host_f64(out[0]) == 0).all()


def test_mfma_decode_full_size_group8_single_pass_equals_split_k():
    """Batch 32, ctx 4096, 64 q / 8 kv heads (group 8), bf16, shuffled pool:
    single pass and split-K agree and two sequences match the oracle."""
    S, H, n_kv, D, BS, L = 32, 64, 8, 128, 16, 4096
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
    for pt in (-1, 512, 0):
        desc = tla.make_decode_desc(q, k, tables, n_kv, scale, partition_tokens=pt)
        ws = torch.empty(max(16, tla.workspace_bytes(desc, L)), dtype=torch.uint8, device="cuda")
        out = torch.empty_like(q)
        print(f"case mfma2 full-size pt={pt}", flush=True)
        tla.paged_attention_decode(desc, out, q, k, v, tables, sl, L, ws)
        torch.cuda.synchronize()
        outs[pt] = out.float()
    for pt in (512, 0):
        assert (outs[pt] - outs[-1]).abs().max().item() <= 2 * ATOL
    tb = tables.cpu().numpy()
    for s in (0, 31):
        blocks = tb[s]
        sub_k = k[blocks.tolist()].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
        sub_v = v[blocks.tolist()].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
        qs = q[s:s + 1].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
        ref = orc.paged_attention(qs, orc.BF16, sub_k, sub_v, orc.BF16, np.arange(nb, dtype=np.int32)[None],
                                  np.array([L], np.int32), n_kv, scale, orc.GROUPED)
        assert_close(outs[-1][s:s + 1].to(torch.bfloat16), ref, orc.BF16, ATOL, f"seq {s}")


def test_mfma_decode_graph_replay_matches_eager():
    """Split-K 2-byte matrix-core decode captured in a HIP graph, replayed
    with eager work between: bit-equal to the eager launch."""
    case = inputs.make_paged_case(63, 6, 64, 8, 128, 16, [4096, 1000, 17, 1, 0, 2047], orc.BF16)
    q, k, v = dev(case.q, case.code), dev(case.k_cache, case.code), dev(case.v_cache, case.code)
    bt, sl = dev(case.tables), dev(case.seq_lens)
    desc = tla.make_decode_desc(q, k, bt, 8, case.scale, partition_tokens=512)
    ws = torch.empty(max(16, tla.workspace_bytes(desc, 4096)), dtype=torch.uint8, device="cuda")
    out = torch.zeros_like(q)
    print("case mfma2 graph replay", flush=True)
    tla.paged_attention_decode(desc, out, q, k, v, bt, sl, 4096, ws)
    torch.cuda.synchronize()
    eager = out.clone()
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    with torch.cuda.graph(graph, stream=cap):
        tla.paged_attention_decode(desc, out, q, k, v, bt, sl, 4096, ws, cap)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        tla.paged_attention_decode(desc, out, q, k, v, bt, sl, 4096, ws)
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
