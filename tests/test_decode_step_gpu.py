"""tl_paged_attention_decode_step: reshape_and_cache of the step's token then
the decode, against the oracle.

The pools after the call must equal orc.reshape_and_cache's bit for bit
(the slot's bytes written, every other byte kept), and the output must
match orc.paged_attention over those pools (max-abs 2e-3 for 2-byte pools,
1e-2 for FP8, each plus half an output ulp).  The call runs the append and
the decode as two launches; FP8 pools take the quantising append."""
import numpy as np
import pytest
import torch

import inputs
import oracle_lib as orc
import tl_attn as tla
from gpu_util import assert_close, dev, host_bits

pytestmark = pytest.mark.gpu

ATOL = 2e-3
ATOL_FP8 = 1e-2
NAN_BITS = {orc.F16: 0x7E00, orc.BF16: 0x7FC0}


def _step_case(seed, lens, H, n_kv, D, BS, code, holes=0):
    """A pool holding tokens 0 .. L - 2 of each sequence (NaN in the new
    token's slot, which the step overwrites), the step's key / value rows
    and the slots of position L - 1."""
    case = inputs.make_paged_case(seed, len(lens), H, n_kv, D, BS, lens, code, holes=holes)
    S = len(lens)
    pos = np.asarray(lens, np.int64) - 1
    slots = np.full(S, -1, np.int32)
    for s in range(S):
        if pos[s] < 0:
            continue
        blk = case.tables[s, pos[s] // BS]
        if blk >= 0:
            slots[s] = blk * BS + pos[s] % BS
            case.k_cache[blk, :, :, pos[s] % BS] = NAN_BITS.get(code, 0)
            case.v_cache[blk, :, :, pos[s] % BS] = NAN_BITS.get(code, 0)
    rng = np.random.default_rng(seed + 3)
    knew = inputs.encode(rng.standard_normal((S, n_kv, D), dtype=np.float32), code)
    vnew = inputs.encode(rng.standard_normal((S, n_kv, D), dtype=np.float32), code)
    return case, knew, vnew, slots


def _run_step(case, knew, vnew, slots, gqa, pt, code):
    q, k, v = dev(case.q, code), dev(case.k_cache, code), dev(case.v_cache, code)
    bt, sl = dev(case.tables), dev(case.seq_lens)
    max_ctx = int(case.seq_lens.max())
    desc = tla.make_decode_desc(q, k, bt, case.num_kv_heads, case.scale, gqa_map=gqa, partition_tokens=pt)
    ws = torch.empty(max(16, tla.workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
    out = torch.full_like(q, float("nan"))
    tla.paged_attention_decode_step(desc, out, q, dev(knew, code), dev(vnew, code), dev(slots), k, v, bt, sl, max_ctx,
                                    ws)
    torch.cuda.synchronize()
    return out, k, v


def _check(case, knew, vnew, slots, gqa, pt, code, atol=ATOL):
    out, k, v = _run_step(case, knew, vnew, slots, gqa, pt, code)
    orc.reshape_and_cache(knew, vnew, case.k_cache, case.v_cache, slots)
    assert np.array_equal(host_bits(k), case.k_cache) and np.array_equal(host_bits(v), case.v_cache)
    ref = orc.paged_attention(case.q, code, case.k_cache, case.v_cache, code, case.tables, case.seq_lens,
                              case.num_kv_heads, case.scale, gqa)
    assert_close(out, ref, code, atol, f"pt={pt} gqa={gqa}")


LENS = [1, 2, 16, 17, 33, 300, 1025, 4100]


@pytest.mark.parametrize("code", [orc.F16, orc.BF16])
@pytest.mark.parametrize("BS", [16, 32])
@pytest.mark.parametrize("pt", [-1, 512, 0])
def test_step_matches_append_then_decode(code, BS, pt):
    """Single pass, 512-token split-K and the library's plan; lengths across
    block and partition edges, the one-token sequence included; a table hole
    inside one sequence."""
    for gqa in (tla.GQA_GROUPED, tla.GQA_MODULO):
        case, knew, vnew, slots = _step_case(200 + BS, LENS, 32, 8, 128, BS, code, holes=1)
        print(f"case decode step code={code} bs={BS} pt={pt} gqa={gqa}", flush=True)
        _check(case, knew, vnew, slots, gqa, pt, code)


def test_step_negative_slot_reads_the_pool():
    """slot -1: nothing is written and position L - 1 comes from the pool, as
    reshape_and_cache (which skips it) then the decode give."""
    case, knew, vnew, slots = _step_case(211, [100, 700, 65], 32, 8, 128, 16, orc.BF16)
    rng = np.random.default_rng(5)
    for s in (1,):                                # a real value at the slot the step will not write
        L = int(case.seq_lens[s])
        blk = case.tables[s, (L - 1) // 16]
        case.k_cache[blk, :, :, (L - 1) % 16] = inputs.encode(rng.standard_normal((8, 128), dtype=np.float32),
                                                              orc.BF16)
        case.v_cache[blk, :, :, (L - 1) % 16] = inputs.encode(rng.standard_normal((8, 128), dtype=np.float32),
                                                              orc.BF16)
        slots[s] = -1
    print("case decode step negative slot", flush=True)
    _check(case, knew, vnew, slots, tla.GQA_GROUPED, 0, orc.BF16)


@pytest.mark.parametrize("H,n_kv", [(64, 2), (8, 8), (64, 8)])
def test_step_head_slices_and_groups(H, n_kv):
    """Groups of 32, 1 and 8."""
    case, knew, vnew, slots = _step_case(220 + H + n_kv, [513, 2048, 77], H, n_kv, 128, 16, orc.F16)
    print(f"case decode step H={H} n_kv={n_kv}", flush=True)
    _check(case, knew, vnew, slots, tla.GQA_GROUPED, 512, orc.F16)


def test_step_head_64():
    """Head size 64 (the dot-product decode)."""
    case, knew, vnew, slots = _step_case(230, [1, 40, 900], 16, 4, 64, 16, orc.F16)
    print("case decode step head 64", flush=True)
    _check(case, knew, vnew, slots, tla.GQA_MODULO, 0, orc.F16)


def test_step_fp8_pool():
    """FP8 pool: the token's bf16 rows quantised with the descriptor's scales
    (tl_reshape_and_cache_fp8), then the FP8 decode."""
    lens = [3, 600, 2049]
    base = inputs.make_paged_case(240, len(lens), 32, 8, 128, 16, lens, orc.F32)
    ks = float(np.abs(base.k_cache).max()) / 448.0
    vs = float(np.abs(base.v_cache).max()) / 448.0
    k8 = orc.f32_to_e4m3(base.k_cache, np.float32(1.0) / np.float32(ks))
    v8 = orc.f32_to_e4m3(base.v_cache, np.float32(1.0) / np.float32(vs))
    q = inputs.encode(orc.bits_to_f32(base.q, orc.F32), orc.BF16)
    rng = np.random.default_rng(7)
    S = len(lens)
    knew = inputs.encode(rng.standard_normal((S, 8, 128), dtype=np.float32), orc.BF16)
    vnew = inputs.encode(rng.standard_normal((S, 8, 128), dtype=np.float32), orc.BF16)
    slots = np.array([base.tables[s, (L - 1) // 16] * 16 + (L - 1) % 16 for s, L in enumerate(lens)], np.int32)
    kd, vd = torch.from_numpy(k8.copy()).cuda(), torch.from_numpy(v8.copy()).cuda()
    qd, bt, sl = dev(q, orc.BF16), dev(base.tables), dev(base.seq_lens)
    desc = tla.make_decode_desc(qd, kd, bt, 8, base.scale, kv_dtype=tla.FP8_E4M3, k_scale=ks, v_scale=vs)
    ws = torch.empty(max(16, tla.workspace_bytes(desc, 2049)), dtype=torch.uint8, device="cuda")
    out = torch.full_like(qd, float("nan"))
    print("case decode step fp8 pool", flush=True)
    tla.paged_attention_decode_step(desc, out, qd, dev(knew, orc.BF16), dev(vnew, orc.BF16), dev(slots), kd, vd, bt,
                                    sl, 2049, ws)
    torch.cuda.synchronize()
    orc.reshape_and_cache_fp8(knew, vnew, orc.BF16, k8, v8, slots, ks, vs)
    assert np.array_equal(kd.cpu().numpy(), k8) and np.array_equal(vd.cpu().numpy(), v8)
    ref = orc.paged_attention(q, orc.BF16, k8, v8, orc.FP8, base.tables, base.seq_lens, 8, base.scale, orc.GROUPED,
                              0, ks, vs)
    assert_close(out, ref, orc.BF16, ATOL_FP8, "fp8 pool")
