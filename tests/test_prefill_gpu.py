"""Chunked prefill (+ decode rows in the same launch) on the GPU against the
oracle's fp64 causal attention (oracle/tl_oracle.c orc_chunked_prefill).

Tolerance: max-abs 2e-3 plus half an output ulp.  P V runs on f16 for both
input types (the weights as one f16 term; a bf16 V staged as f16 times
2^-7)."""
import math

import numpy as np
import pytest
import torch

import inputs
import oracle_lib as orc
import tl_attn as tla
from gpu_util import assert_close, dev

pytestmark = pytest.mark.gpu

ATOL = 2e-3


class PrefillCase:
    """Sequences given as (q_len, seq_len) pairs over one shuffled pool."""

    def __init__(self, seed, shape, H, n_kv, code, BS=16, holes=0, nan_unused=False):
        self.q_lens = np.array([a for a, _ in shape], np.int32)
        self.lens = np.array([b for _, b in shape], np.int32)
        assert (self.q_lens <= self.lens).all()
        S = len(shape)
        self.case = inputs.make_paged_case(seed, S, H, n_kv, 128, BS, self.lens, code, holes=holes)
        if nan_unused:
            nan = 0x7FC0 if code == orc.BF16 else 0x7E00
            for s, L in enumerate(self.lens):
                if L % BS:
                    last = self.case.tables[s, (L - 1) // BS]
                    if last >= 0:
                        self.case.k_cache[last, :, :, L % BS:] = nan
                        self.case.v_cache[last, :, :, L % BS:] = nan
        self.cu = np.concatenate([[0], np.cumsum(self.q_lens)]).astype(np.int32)
        rng = np.random.default_rng(seed + 7)
        self.q = inputs.encode(rng.standard_normal((int(self.cu[-1]), H, 128), dtype=np.float32), code)
        self.code, self.H, self.n_kv, self.S = code, H, n_kv, S

    def run(self, gqa=tla.GQA_GROUPED):
        c = self.case
        q = dev(self.q, self.code)
        k, v = dev(c.k_cache, self.code), dev(c.v_cache, self.code)
        bt, sl, cu = dev(c.tables), dev(self.lens), dev(self.cu)
        out = torch.full_like(q, float("nan"))
        desc = tla.make_prefill_desc(q, k, bt, self.S, self.n_kv, c.scale, gqa_map=gqa)
        tla.chunked_prefill(desc, out, q, cu, k, v, bt, sl, int(self.q_lens.max()))
        torch.cuda.synchronize()
        return out

    def ref(self, gqa=orc.GROUPED):
        c = self.case
        return orc.chunked_prefill(self.q, self.code, self.cu, c.k_cache, c.v_cache, self.code, c.tables,
                                   self.lens, self.n_kv, c.scale, gqa)


MIXED = [(96, 96), (130, 400), (1, 700), (33, 33), (2, 50), (1, 1), (257, 300), (1, 129)]


@pytest.mark.parametrize("code", [orc.BF16, orc.F16])
@pytest.mark.parametrize("gqa", [tla.GQA_GROUPED, tla.GQA_MODULO])
def test_mixed_batch_matches_oracle(code, gqa):
    pc = PrefillCase(inputs.SEEDS[4], MIXED, 16, 4, code)
    print(f"case prefill mixed code={code} gqa={gqa}", flush=True)
    assert_close(pc.run(gqa), pc.ref(gqa), code, ATOL, "mixed")


@pytest.mark.parametrize("scale_exp", [20, -12])
def test_bf16_values_near_the_f16_stage_range(scale_exp):
    """P V runs on f16, a bf16 V staged as 2^-7 v: V scaled by 2^20 (|v| up
    to about 5 * 2^20, below the 2^23 limit) and by 2^-12 (below 2^-7, where
    the f16 stage is subnormal) against the oracle.  The tolerance is the
    usual relative one, 2e-3 of the values' scale (plus half an output ulp);
    scaled down, plus the stage's absolute bound: the f16 subnormal spacing
    2^-24 of 2^-7 v is 2^-17 of v at most.  Scaled down, the outputs are
    checked to stand well above that tolerance, so that a kernel returning
    zeros (or values off by the stage's full magnitude) fails."""
    pc = PrefillCase(inputs.SEEDS[4] + scale_exp, MIXED, 16, 4, orc.BF16)
    v = orc.bits_to_f32(pc.case.v_cache, orc.BF16) * np.float32(2.0 ** scale_exp)
    pc.case.v_cache = inputs.encode(v, orc.BF16)
    print(f"case bf16 V scaled by 2^{scale_exp}", flush=True)
    atol = ATOL * 2.0 ** scale_exp + (2.0 ** -17 if scale_exp < 0 else 0.0)
    ref = pc.ref()
    if scale_exp < 0:
        assert np.abs(ref).max() > 20 * atol
        assert np.mean(np.abs(ref) > 2 * atol) > 0.5
    assert_close(pc.run(), ref, orc.BF16, atol, f"V x 2^{scale_exp}")


@pytest.mark.parametrize("H,n_kv", [(16, 2), (4, 4), (12, 4)])
def test_group_sizes(H, n_kv):
    pc = PrefillCase(inputs.SEEDS[4] + 1, [(70, 200), (1, 333), (40, 40)], H, n_kv, orc.BF16)
    print(f"case prefill H={H} n_kv={n_kv}", flush=True)
    assert_close(pc.run(), pc.ref(), orc.BF16, ATOL, f"H={H}")


def test_block_size_32_holes_and_nan_unused_slots():
    pc = PrefillCase(inputs.SEEDS[4] + 2, [(50, 300), (1, 250), (17, 77)], 16, 4, orc.F16, BS=32, holes=3,
                     nan_unused=True)
    print("case prefill bs32 holes nan", flush=True)
    assert_close(pc.run(), pc.ref(), orc.F16, ATOL, "bs32")


def test_nan_in_unused_slots_bs16():
    pc = PrefillCase(inputs.SEEDS[4] + 3, [(45, 45), (1, 90), (20, 100)], 8, 2, orc.BF16, nan_unused=True)
    print("case prefill nan bs16", flush=True)
    assert_close(pc.run(), pc.ref(), orc.BF16, ATOL, "nan")


def test_chunked_equals_whole_prompt():
    """A 256-token prompt as one chunk and as four 64-token chunks (each chunk
    sees the previous ones through the pool) gives the same rows."""
    whole = PrefillCase(inputs.SEEDS[4] + 4, [(256, 256)], 16, 2, orc.BF16)
    out_whole = whole.run()
    c = whole.case
    k, v = dev(c.k_cache, orc.BF16), dev(c.v_cache, orc.BF16)
    bt = dev(c.tables)
    parts = []
    for i in range(4):
        q = dev(np.ascontiguousarray(whole.q[64 * i: 64 * (i + 1)]), orc.BF16)
        out = torch.full_like(q, float("nan"))
        desc = tla.make_prefill_desc(q, k, bt, 1, 2, c.scale)
        tla.chunked_prefill(desc, out, q, dev(np.array([0, 64], np.int32)), k, v, bt,
                            dev(np.array([64 * (i + 1)], np.int32)), 64)
        parts.append(out)
    torch.cuda.synchronize()
    chunked = torch.cat(parts)
    assert torch.equal(chunked.view(torch.int16), out_whole.view(torch.int16))


def test_decode_rows_match_decode_kernel():
    """q_len == 1 rows of a prefill call agree with the decode entry point
    (same wavefront code and split)."""
    pc = PrefillCase(inputs.SEEDS[4] + 5, [(1, 1000), (1, 4096), (1, 17)], 32, 8, orc.BF16)
    got = pc.run()
    c = pc.case
    q = dev(pc.q, orc.BF16)
    k, v, bt, sl = dev(c.k_cache, orc.BF16), dev(c.v_cache, orc.BF16), dev(c.tables), dev(pc.lens)
    desc = tla.make_decode_desc(q, k, bt, 8, c.scale, partition_tokens=-1)
    out = torch.full_like(q, float("nan"))
    tla.paged_attention_decode(desc, out, q, k, v, bt, sl, int(pc.lens.max()), None)
    torch.cuda.synchronize()
    assert (got.float() - out.float()).abs().max().item() <= 2 * ATOL
    assert_close(got, pc.ref(), orc.BF16, ATOL, "decode rows")


def test_prefill_first_ordering_matches_unordered():
    """num_prefill_seqs (prefill sequences first) gives the same rows as the
    scan of every sequence."""
    pc = PrefillCase(inputs.SEEDS[4] + 7, [(90, 300), (33, 33), (1, 500), (1, 64), (0, 10)], 16, 4, orc.BF16)
    a = pc.run()
    c = pc.case
    q = dev(pc.q, orc.BF16)
    k, v, bt, sl, cu = dev(c.k_cache, orc.BF16), dev(c.v_cache, orc.BF16), dev(c.tables), dev(pc.lens), dev(pc.cu)
    out = torch.full_like(q, float("nan"))
    desc = tla.make_prefill_desc(q, k, bt, pc.S, 4, c.scale, num_prefill_seqs=2)
    tla.chunked_prefill(desc, out, q, cu, k, v, bt, sl, 90)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), out.view(torch.int16))
    assert_close(out, pc.ref(), orc.BF16, ATOL, "ordered")


def test_config5_shape_spot_checks():
    """H=64, n_kv=8, bf16: two 512-row chunks (prefixes 0 and 1536) plus 8
    decode rows at 2048 in one launch; decode rows and the last 4 queries of
    each chunk against the oracle."""
    shape = [(512, 512), (512, 2048)] + [(1, 2048)] * 8
    pc = PrefillCase(inputs.SEEDS[4] + 6, shape, 64, 8, orc.BF16)
    c = pc.case
    q = dev(pc.q, orc.BF16)
    k, v, bt, sl, cu = dev(c.k_cache, orc.BF16), dev(c.v_cache, orc.BF16), dev(c.tables), dev(pc.lens), dev(pc.cu)
    out = torch.full_like(q, float("nan"))
    desc = tla.make_prefill_desc(q, k, bt, pc.S, 8, c.scale, num_prefill_seqs=2)
    tla.chunked_prefill(desc, out, q, cu, k, v, bt, sl, 512)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    for s in range(len(shape)):
        ql, L = int(pc.q_lens[s]), int(pc.lens[s])
        take = min(ql, 4)
        rows = slice(int(pc.cu[s]) + ql - take, int(pc.cu[s + 1]))
        qs = np.ascontiguousarray(pc.q[rows])
        ref = orc.chunked_prefill(qs, orc.BF16, np.array([0, take], np.int32), c.k_cache, c.v_cache, orc.BF16,
                                  np.ascontiguousarray(c.tables[s:s + 1]), np.array([L], np.int32), 8, c.scale)
        g = torch.from_numpy(got[rows]).to(torch.bfloat16)
        assert_close(g, ref, orc.BF16, ATOL, f"seq {s}")


def test_bench_chunk_full_size():
    """The benchmark's launch at full size: 8 prompts' last 512-token chunk
    at ctx 2048 plus 32 decode rows at ctx 2048, 64/8 heads, bf16, one call.
    Every decode row, and rows spread over each chunk (first, last, both
    sides of the 256-row tile edge, and others), against the oracle."""
    shape = [(512, 2048)] * 8 + [(1, 2048)] * 32
    pc = PrefillCase(inputs.SEEDS[4] + 9, shape, 64, 8, orc.BF16)
    c = pc.case
    q = dev(pc.q, orc.BF16)
    k, v, bt, sl, cu = dev(c.k_cache, orc.BF16), dev(c.v_cache, orc.BF16), dev(c.tables), dev(pc.lens), dev(pc.cu)
    out = torch.full_like(q, float("nan"))
    desc = tla.make_prefill_desc(q, k, bt, pc.S, 8, c.scale, num_prefill_seqs=8)
    print("case prefill bench chunk, full size", flush=True)
    tla.chunked_prefill(desc, out, q, cu, k, v, bt, sl, 512)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    # decode rows: one oracle call over the 32 of them
    d0 = int(pc.cu[8])
    ref = orc.chunked_prefill(np.ascontiguousarray(pc.q[d0:]), orc.BF16, np.arange(33, dtype=np.int32),
                              c.k_cache, c.v_cache, orc.BF16, np.ascontiguousarray(c.tables[8:]),
                              np.full(32, 2048, np.int32), 8, c.scale)
    assert_close(torch.from_numpy(got[d0:]).to(torch.bfloat16), ref, orc.BF16, ATOL, "decode rows")
    # prefill rows: each as a one-row call at its own position
    for s in range(8):
        for i in (0, 1, 31, 32, 37, 100, 255, 256, 300, 447, 510, 511):
            row = int(pc.cu[s]) + i
            pos = 2048 - 512 + i
            ref = orc.chunked_prefill(np.ascontiguousarray(pc.q[row:row + 1]), orc.BF16, np.array([0, 1], np.int32),
                                      c.k_cache, c.v_cache, orc.BF16, np.ascontiguousarray(c.tables[s:s + 1]),
                                      np.array([pos + 1], np.int32), 8, c.scale)
            assert_close(torch.from_numpy(got[row:row + 1]).to(torch.bfloat16), ref, orc.BF16, ATOL,
                         f"seq {s} row {i}")


def test_empty_and_invalid_arguments():
    q = torch.zeros(4, 8, 128, dtype=torch.bfloat16, device="cuda")
    k = torch.zeros(4, 2, 128, 16, dtype=torch.bfloat16, device="cuda")
    bt = torch.zeros(1, 4, dtype=torch.int32, device="cuda")
    desc = tla.make_prefill_desc(q, k, bt, 1, 2, 0.1)
    cu = torch.tensor([0, 0], dtype=torch.int32, device="cuda")
    sl = torch.tensor([0], dtype=torch.int32, device="cuda")
    out = torch.zeros_like(q)
    tla.chunked_prefill(desc, out, q[:0], cu, k, k, bt, sl, 0)          # nothing to do
    bad = tla.make_prefill_desc(q, k, bt, 1, 2, 0.1)
    bad.head_size = 64
    with pytest.raises(tla.TLError) as e:
        tla.chunked_prefill(bad, out, q, cu, k, k, bt, sl, 4)
    assert e.value.code == tla.ERR_NOT_IMPLEMENTED
    for scale in (0.0, -0.1, float("inf"), float("nan")):
        neg = tla.make_prefill_desc(q, k, bt, 1, 2, scale)
        with pytest.raises(tla.TLError) as e:
            tla.chunked_prefill(neg, out, q, cu, k, k, bt, sl, 4)
        assert e.value.code == tla.ERR_INVALID_ARGUMENT


# ---------------------------------------------------------------------------
# every power-of-two block size (CudaEngineConfig.paged_kv_block_size,
# config_schema.h:68) and FP8 E4M3 pools (use_fp8_kv, config_schema.h:72)
# ---------------------------------------------------------------------------

BS_MIXED = [(96, 96), (130, 400), (1, 700), (33, 33), (2, 50), (1, 1), (257, 300), (1, 129), (70, 613)]


@pytest.mark.parametrize("code", [orc.BF16, orc.F16])
@pytest.mark.parametrize("BS", [8, 16, 32, 64, 128, 256])
def test_block_sizes_with_holes_and_nan_unused_slots(BS, code):
    """Prefill rows and decode rows at every block size: table holes (which
    drop their keys) and NaN in the slots past each sequence's end."""
    pc = PrefillCase(inputs.SEEDS[4] + 10 + BS, BS_MIXED, 16, 4, code, BS=BS, holes=4, nan_unused=True)
    print(f"case prefill bs={BS} code={code}", flush=True)
    assert_close(pc.run(), pc.ref(), code, ATOL, f"bs={BS}")


def _fp8_case(seed, shape, H, n_kv, qcode, BS, holes=0):
    """A PrefillCase whose pools are E4M3 codes with per-tensor absmax / 448
    scales (fp8_gemm.cu:82-93), NaN codes in the slots past each sequence's
    end; returns (case, k codes, v codes, k_scale, v_scale) with the case's
    own pools replaced by the dequantised values in fp32 (what the oracle
    attends over)."""
    pc = PrefillCase(seed, shape, H, n_kv, orc.F32, BS=BS, holes=holes)
    pc.q = inputs.encode(pc.q, qcode)
    pc.code = qcode
    c = pc.case
    ks = float(np.abs(c.k_cache).max()) / 448
    vs = float(np.abs(c.v_cache).max()) / 448
    k8, v8 = orc.f32_to_e4m3(c.k_cache, 1 / ks), orc.f32_to_e4m3(c.v_cache, 1 / vs)
    for s, L in enumerate(pc.lens):
        if L % BS:
            last = c.tables[s, (L - 1) // BS]
            if last >= 0:
                k8[last, :, :, L % BS:] = 0x7F
                v8[last, :, :, L % BS:] = 0xFF
    c.k_cache = orc.bits_to_f32(k8, orc.FP8) * np.float32(ks)
    c.v_cache = orc.bits_to_f32(v8, orc.FP8) * np.float32(vs)
    return pc, k8, v8, ks, vs


def _run_fp8(pc, k8, v8, ks, vs, gqa=tla.GQA_GROUPED):
    c = pc.case
    q = dev(pc.q, pc.code)
    k, v = dev(k8), dev(v8)
    bt, sl, cu = dev(c.tables), dev(pc.lens), dev(pc.cu)
    out = torch.full_like(q, float("nan"))
    desc = tla.make_prefill_desc(q, k, bt, pc.S, pc.n_kv, c.scale, gqa_map=gqa, kv_dtype=tla.FP8_E4M3,
                                 k_scale=ks, v_scale=vs)
    tla.chunked_prefill(desc, out, q, cu, k, v, bt, sl, int(pc.q_lens.max()))
    torch.cuda.synchronize()
    return out


def _ref_fp8(pc, gqa=orc.GROUPED):
    c = pc.case
    return orc.chunked_prefill(pc.q, pc.code, pc.cu, c.k_cache, c.v_cache, orc.F32, c.tables, pc.lens, pc.n_kv,
                               c.scale, gqa)


@pytest.mark.parametrize("qcode", [orc.BF16, orc.F16])
@pytest.mark.parametrize("BS", [8, 16, 32, 256])
def test_fp8_pool_against_the_dequantised_pool(BS, qcode):
    """FP8 E4M3 pools (codes staged exactly as the q type for q.k and as f16
    for p.v, k_scale in the score scale, v_scale on the output), prefill rows
    and decode rows, against the oracle over the dequantised pool: max-abs
    1e-2 (the FP8 bar).  Holes and NaN codes past the sequences' ends."""
    pc, k8, v8, ks, vs = _fp8_case(inputs.SEEDS[4] + 20 + BS, BS_MIXED, 16, 4, qcode, BS, holes=3)
    print(f"case prefill fp8 bs={BS} q={qcode}", flush=True)
    assert_close(_run_fp8(pc, k8, v8, ks, vs), _ref_fp8(pc), qcode, 1e-2, f"fp8 bs={BS}")


@pytest.mark.parametrize("gqa", [tla.GQA_GROUPED, tla.GQA_MODULO])
def test_fp8_pool_group_sizes_and_head_maps(gqa):
    for H, n_kv in ((8, 8), (32, 4)):
        pc, k8, v8, ks, vs = _fp8_case(inputs.SEEDS[4] + 30 + H, [(80, 200), (1, 333), (40, 40)], H, n_kv,
                                       orc.BF16, 16)
        print(f"case prefill fp8 H={H} n_kv={n_kv} gqa={gqa}", flush=True)
        assert_close(_run_fp8(pc, k8, v8, ks, vs, gqa), _ref_fp8(pc, gqa), orc.BF16, 1e-2, f"fp8 H={H}")
