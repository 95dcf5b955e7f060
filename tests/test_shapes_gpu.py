"""Decode shapes beyond the headline one, and the paged_attention_v2 drop-in.

- Head size 128 with every power-of-two block size the engine's
  `paged_kv_block_size` may take (config_schema.h:68): 8 .. 256 for 2-byte
  and FP8 pools (FP8 at 16 in test_fp8_gpu.py).
- The reference's other dispatch shapes (paged_attention_v1.cu:198-209): F16
  heads 80 and 96, F32 heads 64 and 256, at block size 16.
- tl_paged_attention_v2 runs the library's plan inside the caller's scratch:
  equal to the auto plan where that is single pass, never writing past the
  scratch the engine sizes (cuda_engine.cpp:273-285,1144).

Tolerance: max-abs 2e-3 (fp16 / bf16 / fp32 KV) or 1e-2 (FP8 KV, against
attention on the dequantised pool), each plus half an output ulp."""
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
NAN_BITS = {orc.F16: 0x7E00, orc.BF16: 0x7FC0}


def _ref(case, gqa):
    return orc.paged_attention(case.q, case.code, case.k_cache, case.v_cache, case.code, case.tables,
                               case.seq_lens, case.num_kv_heads, case.scale, gqa)


def _poison_tails(case, code):
    """NaN in the slots past each sequence's length in its last block."""
    BS = case.k_cache.shape[3]
    for s, L in enumerate(case.seq_lens):
        L = int(L)
        if L == 0:
            continue
        last = case.tables[s, (L - 1) // BS]
        if last >= 0 and L % BS:
            case.k_cache[last, :, :, L % BS:] = NAN_BITS[code]
            case.v_cache[last, :, :, L % BS:] = NAN_BITS[code]


def _decode(case, gqa, pt, kv_dtype=None, k_scale=1.0, v_scale=1.0, q=None, k=None, v=None):
    q = dev(case.q, case.code) if q is None else q
    k = dev(case.k_cache, case.code) if k is None else k
    v = dev(case.v_cache, case.code) if v is None else v
    bt, sl = dev(case.tables), dev(case.seq_lens)
    max_ctx = int(case.seq_lens.max())
    desc = tla.make_decode_desc(q, k, bt, case.num_kv_heads, case.scale, kv_dtype=kv_dtype, gqa_map=gqa,
                                partition_tokens=pt, k_scale=k_scale, v_scale=v_scale)
    ws = torch.empty(max(16, tla.workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
    out = torch.full_like(q, float("nan"))
    tla.paged_attention_decode(desc, out, q, k, v, bt, sl, max_ctx, ws)
    torch.cuda.synchronize()
    return out


LENS = [0, 1, 7, 8, 9, 31, 33, 255, 257, 513, 1500, 4100]


@pytest.mark.parametrize("BS", [8, 16, 32, 64, 128, 256])
@pytest.mark.parametrize("code", [orc.F16, orc.BF16])
@pytest.mark.parametrize("pt", [-1, 512, 0])
def test_head128_block_sizes(BS, code, pt):
    """Ragged lengths across block and iteration edges, table holes, NaN in
    the unused slots of the last blocks.  The short sequences (1 .. 9
    tokens) also pin the precision of the bf16 softmax weights in p.v: one
    bf16 rounding of the weights misses 2e-3 there."""
    case = inputs.make_paged_case(70 + BS, len(LENS), 32, 8, 128, BS, LENS, code, holes=3)
    _poison_tails(case, code)
    for gqa in (tla.GQA_GROUPED, tla.GQA_MODULO):
        print(f"case bs={BS} code={code} pt={pt} gqa={gqa}", flush=True)
        out = _decode(case, gqa, pt)
        assert_close(out, _ref(case, gqa), code, ATOL, f"bs={BS} pt={pt}")
        assert (host_f64(out[0]) == 0).all()


@pytest.mark.parametrize("BS", [8, 32, 256])
def test_head128_block_sizes_group_8_and_mha(BS):
    lens = [700, 2049, 65]
    for H, n_kv in ((64, 8), (8, 8)):
        case = inputs.make_paged_case(80 + BS, 3, H, n_kv, 128, BS, lens, orc.BF16, holes=1)
        print(f"case bs={BS} H={H} n_kv={n_kv}", flush=True)
        assert_close(_decode(case, tla.GQA_GROUPED, 512), _ref(case, tla.GQA_GROUPED), orc.BF16, ATOL,
                     f"bs={BS} H={H}")


@pytest.mark.parametrize("BS", [8, 32, 64, 128, 256])
@pytest.mark.parametrize("q_code", [orc.F16, orc.BF16])
@pytest.mark.parametrize("pt", [-1, 512])
def test_fp8_block_sizes(BS, q_code, pt):
    lens = [1, 63, 65, 511, 2000, 4097]
    base = inputs.make_paged_case(90 + BS, len(lens), 32, 8, 128, BS, lens, orc.F32, holes=2)
    ks = float(np.abs(base.k_cache).max()) / 448.0
    vs = float(np.abs(base.v_cache).max()) / 448.0
    k8 = orc.f32_to_e4m3(base.k_cache, np.float32(1.0) / np.float32(ks))
    v8 = orc.f32_to_e4m3(base.v_cache, np.float32(1.0) / np.float32(vs))
    q = inputs.encode(orc.bits_to_f32(base.q, orc.F32), q_code)
    for s, L in enumerate(lens):                  # NaN codes past the lengths
        last = base.tables[s, (L - 1) // BS]
        if last >= 0 and L % BS:
            k8[last, :, :, L % BS:] = 0x7F
            v8[last, :, :, L % BS:] = 0xFF
    ref = orc.paged_attention(q, q_code, k8, v8, orc.FP8, base.tables, base.seq_lens, 8, base.scale,
                              orc.GROUPED, 0, ks, vs)
    print(f"case fp8 bs={BS} q={q_code} pt={pt}", flush=True)
    out = _decode(base, tla.GQA_GROUPED, pt, kv_dtype=tla.FP8_E4M3, k_scale=ks, v_scale=vs, q=dev(q, q_code),
                  k=torch.from_numpy(k8).cuda(), v=torch.from_numpy(v8).cuda())
    assert_close(out, ref, q_code, ATOL_FP8, f"fp8 bs={BS}")


@pytest.mark.parametrize("BS,fp8,layout", [(32, False, "paged"), (8, False, "flash_paged"), (64, True, "flash_paged"),
                                           (8, True, "paged")])
def test_engine_config_descriptor_decodes(BS, fp8, layout):
    """A decode descriptor set up by tl_engine_apply_config (CudaEngineConfig's
    paged_kv_block_size, use_fp8_kv, attention_layout), run against the
    oracle: the mapping gives the kernels the block size and pool type the
    pool was built with."""
    lens = [1, 64, 700, 2049]
    base = inputs.make_paged_case(150 + BS, len(lens), 32, 8, 128, BS, lens, orc.F32 if fp8 else orc.BF16, holes=1)
    bt, sl = dev(base.tables), dev(base.seq_lens)
    if fp8:
        ks = float(np.abs(base.k_cache).max()) / 448.0
        vs = float(np.abs(base.v_cache).max()) / 448.0
        k_np = orc.f32_to_e4m3(base.k_cache, np.float32(1.0) / np.float32(ks))
        v_np = orc.f32_to_e4m3(base.v_cache, np.float32(1.0) / np.float32(vs))
        q_np = inputs.encode(orc.bits_to_f32(base.q, orc.F32), orc.BF16)
        ref = orc.paged_attention(q_np, orc.BF16, k_np, v_np, orc.FP8, base.tables, base.seq_lens, 8, base.scale,
                                  orc.GROUPED, 0, ks, vs)
        q, k, v = dev(q_np, orc.BF16), torch.from_numpy(k_np).cuda(), torch.from_numpy(v_np).cuda()
    else:
        ref = _ref(base, tla.GQA_GROUPED)
        q, k, v = dev(base.q, orc.BF16), dev(base.k_cache, orc.BF16), dev(base.v_cache, orc.BF16)
    # a descriptor made for a bf16 pool at block size 16, then the engine's knobs
    desc = tla.make_decode_desc(q, dev(np.zeros((1, 8, 128, 16), np.uint16), orc.BF16), bt, 8, base.scale,
                                gqa_map=tla.GQA_GROUPED)
    desc.num_blocks = base.k_cache.shape[0]
    tla.engine_apply_config(desc, block_size=BS, use_fp8_kv=fp8, attention_layout=layout)
    assert desc.block_size == BS and desc.kv_dtype == (tla.FP8_E4M3 if fp8 else tla.BF16)
    if fp8:
        desc.k_scale, desc.v_scale = ks, vs
    max_ctx = int(base.seq_lens.max())
    ws = torch.empty(max(16, tla.workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
    out = torch.full_like(q, float("nan"))
    print(f"case engine config bs={BS} fp8={fp8} layout={layout}", flush=True)
    tla.paged_attention_decode(desc, out, q, k, v, bt, sl, max_ctx, ws)
    torch.cuda.synchronize()
    assert_close(out, ref, orc.BF16, ATOL_FP8 if fp8 else ATOL, f"engine config bs={BS}")


@pytest.mark.parametrize("D,code", [(80, orc.F16), (96, orc.F16), (80, orc.BF16), (96, orc.BF16),
                                    (64, orc.F32), (256, orc.F32), (64, orc.BF16), (256, orc.BF16)])
@pytest.mark.parametrize("H,n_kv", [(8, 2), (4, 4)])
def test_reference_dispatch_shapes(D, code, H, n_kv):
    """F16 heads 80 / 96 and F32 heads 64 / 256 at block size 16, through
    the v1 operator (single pass) and split-K; bf16 at the same heads (the
    short sequences check the bf16 weights' precision)."""
    lens = [1, 3, 7, 17, 600, 1300]
    case = inputs.make_paged_case(100 + D, len(lens), H, n_kv, D, 16, lens, code, holes=1)
    if code != orc.F32:
        _poison_tails(case, code)
    q, k, v, bt, sl = (dev(case.q, code), dev(case.k_cache, code), dev(case.v_cache, code), dev(case.tables),
                       dev(case.seq_lens))
    for gqa in (tla.GQA_MODULO, tla.GQA_GROUPED):
        ref = _ref(case, gqa)
        out = torch.full_like(q, float("nan"))
        print(f"case v1 D={D} code={code} H={H} n_kv={n_kv} gqa={gqa}", flush=True)
        tla.paged_attention_v1(out, q, k, v, bt, sl, n_kv, case.scale, D, 16, gqa_map=gqa)
        torch.cuda.synchronize()
        assert_close(out, ref, code, ATOL, f"v1 D={D}")
        print(f"case split-K D={D} code={code} H={H} n_kv={n_kv} gqa={gqa}", flush=True)
        assert_close(_decode(case, gqa, 512), ref, code, ATOL, f"split-K D={D}")


@pytest.mark.parametrize("D,code", [(96, orc.BF16), (256, orc.BF16), (128, orc.F16)])
def test_merge_of_9_to_256_partitions(D, code):
    """Split-K into 9-19 partitions of 512 tokens (the wide log-sum-exp
    merge, whose loads all start before the sequence length is read):
    ragged lengths with an empty sequence, holes and NaN tails, against the
    oracle."""
    lens = [9000, 1, 4600, 0, 513, 6001]
    case = inputs.make_paged_case(300 + D, len(lens), 8, 2, D, 16, lens, code, holes=2)
    _poison_tails(case, code)
    for gqa in (tla.GQA_MODULO, tla.GQA_GROUPED):
        print(f"case wide merge D={D} code={code} gqa={gqa}", flush=True)
        assert_close(_decode(case, gqa, 512), _ref(case, gqa), code, ATOL, f"wide merge D={D}")


def test_merge_of_more_than_256_partitions():
    """One sequence of 133 000 tokens (32/8 heads, d 128, bf16): 260
    partitions of 512 tokens (the long merge), 65 of 2048 (the wide merge)
    and the single pass agree."""
    L, H, n_kv, D, BS = 133000, 32, 8, 128, 16
    g = torch.Generator(device="cuda").manual_seed(inputs.SEEDS[2])
    nb = (L + BS - 1) // BS
    N = nb + 7
    tables = torch.randperm(N, generator=g, device="cuda").to(torch.int32)[:nb].view(1, nb).contiguous()
    k = torch.randn(N, n_kv, D, BS, generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn(N, n_kv, D, BS, generator=g, device="cuda").to(torch.bfloat16)
    q = torch.randn(1, H, D, generator=g, device="cuda").to(torch.bfloat16)
    sl = torch.tensor([L], dtype=torch.int32, device="cuda")
    outs = {}
    for pt in (-1, 512, 2048):
        desc = tla.make_decode_desc(q, k, tables, n_kv, 1 / math.sqrt(D), partition_tokens=pt)
        ws = torch.empty(max(16, tla.workspace_bytes(desc, L)), dtype=torch.uint8, device="cuda")
        out = torch.full_like(q, float("nan"))
        print(f"case long merge pt={pt}", flush=True)
        tla.paged_attention_decode(desc, out, q, k, v, tables, sl, L, ws)
        torch.cuda.synchronize()
        outs[pt] = out.float()
    for pt in (512, 2048):
        assert (outs[pt] - outs[-1]).abs().max().item() <= 2 * ATOL, pt


# ---------------------------------------------------------------------------
# paged_attention_v2 drop-in
# ---------------------------------------------------------------------------

GUARD = 4096


def _v2_guarded(case, code, stream=None, kernel_sizing=False, capacity=None):
    """tl_paged_attention_v2 with the engine's scratch sizes (or, with
    kernel_sizing, the partition count the reference kernel itself writes,
    paged_attention_v2.cu:196; with capacity, a scratch of that many
    partitions through tl_paged_attention_v2_capacity) followed by sentinel
    guards; returns (out, guards intact)."""
    q, k, v, bt, sl = (dev(case.q, code), dev(case.k_cache, code), dev(case.v_cache, code), dev(case.tables),
                       dev(case.seq_lens))
    S, H, D = q.shape
    BS = k.shape[3]
    max_ctx = int(case.seq_lens.max())
    P = (max_ctx // BS + 31) // 32 if kernel_sizing else tla.v2_num_partitions(max_ctx, BS)
    if capacity is not None:
        P = capacity
    n = S * H * P
    if n == 0:
        n = 1
    es = torch.full((n + GUARD,), 7.25, dtype=torch.float32, device="cuda")
    ml = torch.full((n + GUARD,), -3.5, dtype=torch.float32, device="cuda")
    tmp = torch.full((n * D + GUARD,), 1.5, dtype=q.dtype, device="cuda")
    out = torch.full_like(q, float("nan"))
    tla.paged_attention_v2(out, es, ml, tmp, q, k, v, bt, sl, case.num_kv_heads, case.scale, D, BS, max_ctx,
                           stream, gqa_map=tla.GQA_MODULO, scratch_partitions=capacity)
    torch.cuda.synchronize()
    intact = bool((es[n:] == 7.25).all() and (ml[n:] == -3.5).all() and (tmp[n * D:] == 1.5).all())
    return out, intact


def test_v2_at_batch_64_is_the_single_pass_kernel():
    """Batch 64, ctx 4096, 32/8 heads, bf16: the plan is single pass, so v2
    gives the bytes of tl_paged_attention_decode's auto plan."""
    case = inputs.make_paged_case(inputs.SEEDS[1], 64, 32, 8, 128, 16, [4096] * 64, orc.BF16)
    print("case v2 B=64 ctx 4096", flush=True)
    a, intact = _v2_guarded(case, orc.BF16)
    assert intact
    b = _decode(case, tla.GQA_MODULO, 0)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    for s in (0, 63):
        sub = inputs.PagedCase(case.q[s:s + 1], case.k_cache, case.v_cache, case.tables[s:s + 1],
                               case.seq_lens[s:s + 1], case.code, 8, case.scale)
        assert_close(a[s:s + 1], _ref(sub, orc.MODULO), orc.BF16, ATOL, f"seq {s}")


@pytest.mark.parametrize("lens,code,BS", [
    ([5000], orc.F16, 16),            # the engine's one-sequence call: capped partitions
    ([529], orc.F16, 16),             # just past the engine's v2 threshold
    ([16384], orc.BF16, 16),
    ([3000, 700, 9000, 1], orc.F16, 16),
    ([6000, 100], orc.F32, 16),       # 4-byte tmp_out: as many fp32 partitions as the engine's
    ([5000, 33], orc.BF16, 64),
])
def test_v2_split_k_stays_inside_the_callers_scratch(lens, code, BS):
    D = 128
    case = inputs.make_paged_case(110 + len(lens), len(lens), 32, 8, D, BS, lens, code)
    print(f"case v2 lens={lens} code={code} bs={BS}", flush=True)
    out, intact = _v2_guarded(case, code)
    assert intact, "v2 wrote past the caller's scratch"
    assert_close(out, _ref(case, orc.MODULO), code, ATOL, f"v2 {lens}")


@pytest.mark.parametrize("lens,code,BS", [
    ([1541], orc.F16, 16),            # engine count 4, kernel count 3
    ([1541, 900], orc.F16, 16),
    ([1537, 17], orc.BF16, 16),       # 4 against 3
    ([1030], orc.F16, 32),            # 2 against 1: a single fp32 slot, single pass
    ([4111], orc.F32, 16),            # 9 against 8, 4-byte tmp_out
])
def test_v2_stays_inside_scratch_sized_by_the_reference_kernel(lens, code, BS):
    """A caller that sizes exp_sums / max_logits / tmp_out by the partition
    count of the reference kernel, (max_ctx / bs + 31) / 32, which is one
    less than the engine's ceiling count at these lengths."""
    case = inputs.make_paged_case(130 + len(lens), len(lens), 32, 8, 128, BS, lens, code)
    print(f"case v2 kernel-sized scratch lens={lens} code={code} bs={BS}", flush=True)
    out, intact = _v2_guarded(case, code, kernel_sizing=True)
    assert intact, "v2 wrote past the caller's scratch"
    assert_close(out, _ref(case, orc.MODULO), code, ATOL, f"v2 {lens}")


@pytest.mark.parametrize("lens,code,cap", [
    ([4096], orc.F16, 16),            # the engine's scratch for n_ctx_train 8192: 16 x 256 tokens
    ([4096], orc.F16, 64),            # room for the library plan: 32 x 128
    ([4097], orc.BF16, 16),           # fp32 partials in 16 slots' bytes
    ([3000, 1200], orc.F16, 40),
    ([700], orc.F32, 9),
])
def test_v2_capacity_stays_inside_the_allocated_scratch(lens, code, cap):
    """tl_paged_attention_v2_capacity with a scratch allocated for cap
    partitions (more than the call's context needs): against the oracle,
    the guards past the allocation intact, and the plan the one reported."""
    case = inputs.make_paged_case(140 + len(lens) + cap, len(lens), 32, 8, 128, 16, lens, code)
    P, _ = tla.v2_plan(len(lens), 32, 8, 128, 16, code, int(max(lens)), scratch_partitions=cap)
    print(f"case v2 capacity lens={lens} code={code} cap={cap} P={P}", flush=True)
    out, intact = _v2_guarded(case, code, capacity=cap)
    assert intact, "v2 wrote past the allocated scratch"
    assert_close(out, _ref(case, orc.MODULO), code, ATOL, f"v2 capacity {lens}")


def test_v2_misaligned_scratch_runs_single_pass():
    """A tmp_out that is not 16-byte aligned is not used: the call runs
    single pass and leaves the scratch as it was."""
    case = inputs.make_paged_case(120, 2, 32, 8, 128, 16, [3000, 4000], orc.F16)
    q, k, v, bt, sl = (dev(case.q, orc.F16), dev(case.k_cache, orc.F16), dev(case.v_cache, orc.F16),
                       dev(case.tables), dev(case.seq_lens))
    P = tla.v2_num_partitions(4000, 16)
    es = torch.full((2 * 32 * P,), 7.25, dtype=torch.float32, device="cuda")
    ml = torch.full((2 * 32 * P,), -3.5, dtype=torch.float32, device="cuda")
    big = torch.full((2 * 32 * P * 128 + 8,), 1.5, dtype=torch.float16, device="cuda")
    tmp = big[1:]                                  # 2-byte offset
    out = torch.full_like(q, float("nan"))
    print("case v2 misaligned tmp_out", flush=True)
    tla.paged_attention_v2(out, es, ml, tmp, q, k, v, bt, sl, 8, case.scale, 128, 16, 4000, gqa_map=tla.GQA_MODULO)
    torch.cuda.synchronize()
    assert (es == 7.25).all() and (ml == -3.5).all() and (big == 1.5).all()
    assert_close(out, _ref(case, orc.MODULO), orc.F16, ATOL, "v2 misaligned")
