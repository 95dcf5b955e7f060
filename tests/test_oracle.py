"""Pins the CPU oracle before it is trusted as the checker.

Each check is chosen so that a plausible mistake in the oracle (a wrong
rounding rule, a swapped index in the block-table gather, a dropped
softmax term, a wrong GQA mapping, a mis-packed nibble) fails it:
  - conversions against independent implementations (numpy float16, torch
    bfloat16 / float8_e4m3fn) and brute force over every code;
  - attention against a vectorised numpy float64 implementation on small
    inputs, plus closed forms (L = 1 gives v, constant K gives mean(V)) and
    invariants (split-K + LSE = single pass, physical-block permutation,
    holes = removed tokens);
  - the KIVI codec against the known answers and bounds of the reference's
    own tests (test_kivi_bounds.cpp, test_kivi_roundtrip.cpp) and a
    hand-derived record.
"""
import math

import numpy as np
import pytest
import torch

import golden_cases
import inputs
import oracle_lib as orc


# ---------------------------------------------------------------------------
# conversions
# ---------------------------------------------------------------------------

def test_f16_decode_all_codes_matches_numpy():
    codes = np.arange(65536, dtype=np.uint16)
    got = orc.bits_to_f32(codes, orc.F16)
    want = codes.view(np.float16).astype(np.float32)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()


def test_f16_encode_matches_numpy_rne():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * 10,
        (rng.standard_normal(50000) * 1e-5).astype(np.float32),      # subnormal range
        np.array([65504, 65519.99, 65520, 1e6, -1e6, 0.0, -0.0, np.inf, -np.inf], np.float32),
        # exact halfway points between adjacent fp16 values (ties to even)
        ((np.arange(1024, 2048, dtype=np.float32) + 0.5) * 2.0 ** -10),
        ((np.arange(0, 1024, dtype=np.float32) + 0.5) * 2.0 ** -24),
    ]).astype(np.float32)
    got = orc.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_bf16_encode_matches_torch_rne():
    rng = np.random.default_rng(2)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * 100,
        np.array([0.0, -0.0, np.inf, -np.inf, 3.3895314e38], np.float32),
        (np.arange(0, 4096, dtype=np.uint32) * 65536 + 32768).view(np.float32),  # ties
    ]).astype(np.float32)
    got = orc.f32_to_bf16_bits(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


def _e4m3_values():
    return torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()


def test_e4m3_decode_all_codes_matches_torch():
    got = orc.bits_to_f32(np.arange(256, dtype=np.uint8), orc.FP8)
    want = _e4m3_values()
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok], want[ok])
    assert got[0x7E] == 448.0 and np.isnan(got[0x7F]) and np.isnan(got[0xFF])


def test_e4m3_encode_every_f16_brute_force():
    """RNE to the nearest finite E4M3 value (ties to even code), saturate at
    448: brute force over all 256 codes for every fp16 input."""
    x = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    x = x[np.isfinite(x)]
    vals = orc.bits_to_f32(np.arange(256, dtype=np.uint8), orc.FP8).astype(np.float64)
    finite = np.where(~np.isnan(vals))[0]
    got = orc.f32_to_e4m3(x)
    # nearest by distance, ties to the even mantissa (code with bit0 == 0)
    xv = x.astype(np.float64)[:, None]
    dist = np.abs(xv - vals[finite][None, :])
    dmin = dist.min(axis=1, keepdims=True)
    cand = (dist == dmin)
    codes = finite[None, :].repeat(len(x), 0)
    even = cand & ((codes & 1) == 0)
    pick_even = even.any(axis=1)
    idx = np.where(pick_even, np.argmax(even, axis=1), np.argmax(cand, axis=1))
    want = finite[idx].astype(np.uint8)
    # a result of zero keeps the sign of the input (IEEE rounding)
    want = np.where((vals[want] == 0) & np.signbit(x), 0x80, want).astype(np.uint8)
    sat = np.abs(x) >= 448
    want = np.where(sat, np.where(x < 0, 0xFE, 0x7E), want).astype(np.uint8)
    assert np.array_equal(got, want)


def test_e4m3_encode_matches_torch_in_range():
    x = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    x = x[np.isfinite(x) & (np.abs(x) < 464)]
    got = orc.f32_to_e4m3(x)
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got, want)
    assert orc.lib.orc_f32_to_e4m3(float("inf")) == 0x7E
    assert orc.lib.orc_f32_to_e4m3(-1e9) == 0xFE
    assert orc.lib.orc_f32_to_e4m3(float("nan")) & 0x7F == 0x7F


# ---------------------------------------------------------------------------
# reshape_and_cache
# ---------------------------------------------------------------------------

def test_reshape_and_cache_index_map():
    T, n_kv, D, BS, N = 5, 3, 8, 4, 6
    key = np.arange(T * n_kv * D, dtype=np.uint16).reshape(T, n_kv, D)
    val = (key + 1000).astype(np.uint16)
    kc = np.zeros((N, n_kv, D, BS), np.uint16)
    vc = np.zeros_like(kc)
    slots = np.array([0, 7, -1, 23, 13], np.int32)
    orc.reshape_and_cache(key, val, kc, vc, slots)
    for t, s in enumerate(slots):
        if s < 0:
            continue
        assert np.array_equal(kc[s // BS, :, :, s % BS], key[t])
        assert np.array_equal(vc[s // BS, :, :, s % BS], val[t])
    # nothing else written: the skipped token's data appears nowhere
    assert not np.isin(key[2], kc).any()
    assert (kc != 0).sum() == 4 * n_kv * D - 1  # element 0 of token 0 is 0 itself


def test_reshape_then_gather_roundtrip():
    """gather(scatter(x)) == x through slot = table[pos // BS] * BS + pos % BS
    (cuda_allocator.cpp:270-274)."""
    rng = np.random.default_rng(3)
    n_kv, D, BS, N, L = 2, 16, 16, 20, 70
    table = rng.permutation(N)[: (L + BS - 1) // BS].astype(np.int32)
    pos = np.arange(L)
    slots = (table[pos // BS] * BS + pos % BS).astype(np.int32)
    key = rng.integers(0, 65535, (L, n_kv, D), dtype=np.uint16)
    kc = np.zeros((N, n_kv, D, BS), np.uint16)
    vc = np.zeros_like(kc)
    orc.reshape_and_cache(key, key, kc, vc, slots)
    back = kc[table[pos // BS], :, :, pos % BS]
    assert np.array_equal(back, key)


# ---------------------------------------------------------------------------
# paged attention
# ---------------------------------------------------------------------------

def numpy_attention(case: inputs.PagedCase, gqa_map):
    """Vectorised float64 restatement used to cross-check the C loops."""
    S, H, D, BS = case.shape
    q = orc.bits_to_f32(case.q, case.code).astype(np.float64) if case.code != orc.F32 else case.q.astype(np.float64)
    kc = orc.bits_to_f32(case.k_cache, case.code).astype(np.float64) if case.code != orc.F32 else case.k_cache.astype(np.float64)
    vc = orc.bits_to_f32(case.v_cache, case.code).astype(np.float64) if case.code != orc.F32 else case.v_cache.astype(np.float64)
    G = H // case.num_kv_heads
    out = np.zeros((S, H, D))
    for s in range(S):
        L = int(case.seq_lens[s])
        if L == 0:
            continue
        pos = np.arange(L)
        phys = case.tables[s][pos // BS]
        keep = phys >= 0
        pos, phys = pos[keep], phys[keep]
        for h in range(H):
            kvh = h // G if gqa_map == orc.GROUPED else h % case.num_kv_heads
            K = kc[phys, kvh, :, pos % BS]          # [L, D]
            V = vc[phys, kvh, :, pos % BS]
            sc = K @ q[s, h] * float(np.float32(case.scale))
            w = np.exp(sc - sc.max())
            out[s, h] = (w / w.sum()) @ V
    return out


@pytest.mark.parametrize("gqa_map", [orc.MODULO, orc.GROUPED])
@pytest.mark.parametrize("code", [orc.F16, orc.BF16, orc.F32])
def test_attention_matches_numpy(gqa_map, code):
    case = inputs.make_paged_case(11, S=3, H=8, n_kv=2, D=32, BS=16, lens=[1, 40, 77], code=code)
    got = orc.paged_attention(case.q, code, case.k_cache, case.v_cache, code, case.tables,
                              case.seq_lens, 2, case.scale, gqa_map)
    np.testing.assert_allclose(got, numpy_attention(case, gqa_map), rtol=0, atol=1e-12)


def test_attention_single_token_returns_v():
    case = inputs.make_paged_case(12, S=2, H=4, n_kv=4, D=16, BS=16, lens=[1, 1], code=orc.F16)
    got = orc.paged_attention(case.q, orc.F16, case.k_cache, case.v_cache, orc.F16, case.tables,
                              case.seq_lens, 4, case.scale, orc.GROUPED)
    for s in range(2):
        b = case.tables[s, 0]
        want = orc.bits_to_f32(case.v_cache[b, :, :, 0], orc.F16)
        np.testing.assert_array_equal(got[s], want)


def test_attention_constant_keys_give_mean_of_values():
    case = inputs.make_paged_case(13, S=1, H=2, n_kv=1, D=16, BS=16, lens=[37], code=orc.F32)
    case.k_cache[:] = 0.25                          # every score equal
    got = orc.paged_attention(case.q, orc.F32, case.k_cache, case.v_cache, orc.F32, case.tables,
                              case.seq_lens, 1, case.scale, orc.GROUPED)
    pos = np.arange(37)
    V = case.v_cache[case.tables[0][pos // 16], 0, :, pos % 16].astype(np.float64)
    np.testing.assert_allclose(got[0, 0], V.mean(0), atol=1e-12)
    np.testing.assert_allclose(got[0, 1], V.mean(0), atol=1e-12)


@pytest.mark.parametrize("pt", [16, 48, 512])
def test_split_k_lse_equals_single_pass(pt):
    lens = inputs.uniform_lens(5, 4, 1, 1200)
    case = inputs.make_paged_case(14, S=4, H=4, n_kv=2, D=32, BS=16, lens=lens, code=orc.BF16)
    a = orc.paged_attention(case.q, orc.BF16, case.k_cache, case.v_cache, orc.BF16, case.tables,
                            case.seq_lens, 2, case.scale, orc.GROUPED, 0)
    b = orc.paged_attention(case.q, orc.BF16, case.k_cache, case.v_cache, orc.BF16, case.tables,
                            case.seq_lens, 2, case.scale, orc.GROUPED, pt)
    np.testing.assert_allclose(a, b, atol=1e-12)


def test_physical_block_permutation_invariance():
    case = inputs.make_paged_case(15, S=2, H=4, n_kv=2, D=16, BS=16, lens=[100, 33], code=orc.F16)
    a = orc.paged_attention(case.q, orc.F16, case.k_cache, case.v_cache, orc.F16, case.tables,
                            case.seq_lens, 2, case.scale, orc.GROUPED)
    N = case.k_cache.shape[0]
    perm = np.random.default_rng(0).permutation(N)
    inv = np.argsort(perm)
    k2 = np.ascontiguousarray(case.k_cache[perm])    # new block i holds old block perm[i]
    v2 = np.ascontiguousarray(case.v_cache[perm])
    t2 = np.where(case.tables >= 0, inv[np.maximum(case.tables, 0)], -1).astype(np.int32)
    b = orc.paged_attention(case.q, orc.F16, k2, v2, orc.F16, t2, case.seq_lens, 2, case.scale,
                            orc.GROUPED)
    np.testing.assert_array_equal(a, b)


def test_table_hole_equals_removed_tokens():
    case = inputs.make_paged_case(16, S=1, H=2, n_kv=1, D=16, BS=16, lens=[48], code=orc.F32)
    with_hole = case.tables.copy()
    with_hole[0, 1] = -1
    a = orc.paged_attention(case.q, orc.F32, case.k_cache, case.v_cache, orc.F32, with_hole,
                            case.seq_lens, 1, case.scale, orc.GROUPED)
    # same tokens without the hole: move block 2 into slot 1 and shorten
    packed = np.full_like(case.tables, -1)
    packed[0, 0], packed[0, 1] = case.tables[0, 0], case.tables[0, 2]
    b = orc.paged_attention(case.q, orc.F32, case.k_cache, case.v_cache, orc.F32, packed,
                            np.array([32], np.int32), 1, case.scale, orc.GROUPED)
    np.testing.assert_allclose(a, b, atol=1e-12)


def test_gqa_mappings_pick_the_right_kv_head():
    case = inputs.make_paged_case(17, S=1, H=8, n_kv=2, D=16, BS=16, lens=[20], code=orc.F32)
    case.v_cache[:, 0] = 1.0
    case.v_cache[:, 1] = 2.0
    g = orc.paged_attention(case.q, orc.F32, case.k_cache, case.v_cache, orc.F32, case.tables,
                            case.seq_lens, 2, case.scale, orc.GROUPED)
    m = orc.paged_attention(case.q, orc.F32, case.k_cache, case.v_cache, orc.F32, case.tables,
                            case.seq_lens, 2, case.scale, orc.MODULO)
    np.testing.assert_allclose(g[0, :, 0], [1, 1, 1, 1, 2, 2, 2, 2])
    np.testing.assert_allclose(m[0, :, 0], [1, 2, 1, 2, 1, 2, 1, 2])


def test_empty_sequence_gives_zeros():
    case = inputs.make_paged_case(18, S=2, H=2, n_kv=1, D=16, BS=16, lens=[0, 5], code=orc.F16)
    got = orc.paged_attention(case.q, orc.F16, case.k_cache, case.v_cache, orc.F16, case.tables,
                              case.seq_lens, 1, case.scale, orc.GROUPED)
    assert (got[0] == 0).all() and (got[1] != 0).any()


def test_fp8_attention_is_attention_on_dequantised_pool():
    case = inputs.make_paged_case(19, S=2, H=4, n_kv=2, D=32, BS=16, lens=[50, 17], code=orc.F32)
    ks, vs = 0.01, 0.02
    k8 = orc.f32_to_e4m3(case.k_cache, 1 / ks)
    v8 = orc.f32_to_e4m3(case.v_cache, 1 / vs)
    got = orc.paged_attention(case.q, orc.F32, k8, v8, orc.FP8, case.tables, case.seq_lens, 2,
                              case.scale, orc.GROUPED, 0, ks, vs)
    kd = (orc.bits_to_f32(k8, orc.FP8).astype(np.float64) * ks).astype(np.float32)
    vd = (orc.bits_to_f32(v8, orc.FP8).astype(np.float64) * vs).astype(np.float32)
    want = orc.paged_attention(case.q, orc.F32, kd, vd, orc.F32, case.tables, case.seq_lens, 2,
                               case.scale, orc.GROUPED)
    np.testing.assert_allclose(got, want, atol=1e-6)


def test_cpu_baseline_f32_matches_oracle():
    lens = inputs.uniform_lens(6, 3, 1, 700)
    case = inputs.make_paged_case(20, S=3, H=8, n_kv=2, D=128, BS=16, lens=lens, code=orc.BF16)
    a = orc.paged_attention(case.q, orc.BF16, case.k_cache, case.v_cache, orc.BF16, case.tables,
                            case.seq_lens, 2, case.scale, orc.GROUPED)
    b = orc.paged_attention_f32(case.q, orc.BF16, case.k_cache, case.v_cache, orc.BF16,
                                case.tables, case.seq_lens, 2, case.scale, orc.GROUPED, threads=4)
    np.testing.assert_allclose(b, a, atol=2e-5)


def test_literal_v1_documents_reference_divergence():
    """The reference kernel's literal output (Appendix-C semantics): dims >=
    block_size are never written (per-thread accumulators are not reduced),
    so it is not attention."""
    case = inputs.make_paged_case(21, S=2, H=4, n_kv=2, D=64, BS=16, lens=[40, 100], code=orc.F16)
    lit = orc.paged_attention_literal_v1(case.q, case.k_cache, case.v_cache, orc.F16, case.tables,
                                         case.seq_lens, 2, case.scale)
    assert (lit[:, :, 16:] == 0).all()
    want = orc.paged_attention(case.q, orc.F16, case.k_cache, case.v_cache, orc.F16, case.tables,
                               case.seq_lens, 2, case.scale, orc.MODULO)
    assert np.abs(lit - want).max() > 0.05


# ---------------------------------------------------------------------------
# chunked prefill
# ---------------------------------------------------------------------------

def test_prefill_last_row_equals_decode_and_chunks_equal_whole():
    rng = np.random.default_rng(22)
    case = inputs.make_paged_case(22, S=1, H=4, n_kv=2, D=32, BS=16, lens=[96], code=orc.BF16)
    qp = inputs.encode(rng.standard_normal((96, 4, 32), dtype=np.float32), orc.BF16)
    whole = orc.chunked_prefill(qp, orc.BF16, np.array([0, 96], np.int32), case.k_cache,
                                case.v_cache, orc.BF16, case.tables, case.seq_lens, 2, case.scale)
    # second half as its own chunk over the full context
    half = orc.chunked_prefill(np.ascontiguousarray(qp[48:]), orc.BF16, np.array([0, 48], np.int32),
                               case.k_cache, case.v_cache, orc.BF16, case.tables, case.seq_lens, 2,
                               case.scale)
    np.testing.assert_allclose(half, whole[48:], atol=1e-12)
    dec = orc.paged_attention(np.ascontiguousarray(qp[95:96]), orc.BF16, case.k_cache,
                              case.v_cache, orc.BF16, case.tables, case.seq_lens, 2, case.scale,
                              orc.GROUPED)
    np.testing.assert_allclose(whole[95:96], dec, atol=1e-12)
    # the first row sees only token 0: its output is v[0]
    b = case.tables[0, 0]
    v0 = orc.bits_to_f32(case.v_cache[b, :, :, 0], orc.BF16)
    np.testing.assert_allclose(whole[0, 0], v0[0], atol=1e-12)
    np.testing.assert_allclose(whole[0, 3], v0[1], atol=1e-12)


# ---------------------------------------------------------------------------
# reference KIVI vector codec
# ---------------------------------------------------------------------------

def test_kivi_known_answers_from_reference_tests():
    # test_kivi_bounds.cpp:27-29, 37-56, 67-68
    assert orc.kivi_compressed_bytes(128, 8, 16) == 24 + 8 * 12
    assert orc.kivi_compressed_bytes(64, 0, 16) == 4 * 12
    assert orc.kivi_compressed_bytes(64, 64, 16) == 64 * 3
    assert orc.kivi_params_supported(128, 8, 16)
    assert orc.kivi_params_supported(64, 4, 16)
    assert orc.kivi_params_supported(128, 64, 16)
    assert not orc.kivi_params_supported(129, 8, 16)
    assert not orc.kivi_params_supported(128, 65, 16)
    assert not orc.kivi_params_supported(16, 32, 16)
    assert not orc.kivi_params_supported(128, 8, 0)
    assert not orc.kivi_params_supported(128, 8, -4)
    assert not orc.kivi_params_supported(0, 0, 16)
    assert not orc.kivi_params_supported(-1, 0, 16)


def _f16(x):
    return np.atleast_1d(np.asarray(x, np.float32)).astype(np.float16).view(np.uint16)


def _roundtrip(x, D, O, G):
    n = x.size // D
    rec = orc.kivi_compress(_f16(x), D, O, G)
    return orc.kivi_decompress(rec, n, D, O, G).view(np.float16).astype(np.float32)


def test_kivi_roundtrip_int4_granularity():
    # test_kivi_roundtrip.cpp:83-113
    x = np.array([[0.1 * d + 0.5 * v for d in range(64)] for v in range(3)], np.float32).ravel()
    got = _roundtrip(x, 64, 0, 16)
    assert np.abs(got - x).max() <= 0.15


def test_kivi_roundtrip_outliers_preserved():
    # test_kivi_roundtrip.cpp:121-170
    x = np.array([0.01 * (i % 64) for i in range(128)], np.float32)
    for v in range(2):
        for k, ch in enumerate([3, 17, 33, 55]):
            x[v * 64 + ch] = 50.0 + k + v
    got = _roundtrip(x, 64, 4, 16)
    assert np.abs(got - x).max() <= 0.1


def test_kivi_degenerate_group_is_constant():
    # test_kivi_roundtrip.cpp:178-200
    got = _roundtrip(np.full(32, 2.5, np.float32), 32, 0, 16)
    assert np.abs(got - 2.5).max() <= 1e-2


def test_kivi_unsupported_params_no_op():
    # test_kivi_roundtrip.cpp:207-229
    stride = orc.kivi_compressed_bytes(256, 0, 16)
    out = np.full(stride, 0xAB, np.uint8)
    orc.kivi_compress(_f16(np.ones(256)), 256, 0, 16, out=out)
    assert (out == 0xAB).all()


def test_kivi_hand_derived_record():
    """x = [1, -3, 0.5, 2], one outlier, group 4: outlier (1, -3); residual
    [1, 0.5, 2] -> gmin 0.5, range 1.5, scale 10 -> q = 5, 0, 15; step
    fp16(0.1) = 0x2E66, zero fp16(0.5) = 0x3800."""
    rec = orc.kivi_compress(_f16([1, -3, 0.5, 2]), 4, 1, 4)
    assert list(rec) == [0x01, 0x00, 0xC2, 0x05, 0x0F, 0x66, 0x2E, 0x00, 0x38]
    back = orc.kivi_decompress(rec, 1, 4, 1, 4).view(np.float16).astype(np.float32)
    assert list(back) == [1.0, -3.0, 0.5, 2.0]


@pytest.mark.parametrize("x,O,G,want", golden_cases.KIVI_SLOT_ORDER_CASES)
def test_kivi_hand_derived_records_keep_slot_order(x, O, G, want):
    D = len(x)
    assert orc.kivi_compressed_bytes(D, O, G) == len(want)
    rec = orc.kivi_compress(_f16(x), D, O, G)
    assert [int(b) for b in rec] == want
    back = orc.kivi_decompress(rec, 1, D, O, G).view(np.float16).astype(np.float32)
    # outliers verbatim; residual codes 0 / 15 at step 1/30 land within one
    # fp16 ulp of the inputs (1 + 15 * fp16(1/30) = 1.49988 -> fp16 1.5)
    assert list(back) == x


def test_kivi_quant_group_nibbles_follow_rne():
    q, st, ze = orc.kivi_quant_group(np.arange(16, dtype=np.float32))
    assert list(q) == list(range(16))
    assert st == int(_f16(1.0)[0]) and ze == 0
    q, st, ze = orc.kivi_quant_group(np.array([0.0, 0.5, 1.0, 2.0], np.float32) * 2)
    # scale = 15/4: (1*3.75 = 3.75 -> 4), (2*3.75 = 7.5 -> 8 even), (4*3.75 = 15)
    assert list(q) == [0, 4, 8, 15]


# ---------------------------------------------------------------------------
# paged KIVI page format
# ---------------------------------------------------------------------------

def test_kivi_page_nibble_positions_are_a_bijection():
    # mark one token/channel at a time: exactly one nibble of the K (V) area moves
    base_k = np.zeros((32, 128), np.float32)
    base_k[0, :] = 1.0                                   # gmin 0, gmax 1 everywhere
    base_v = np.zeros((32, 128), np.float32)
    base_v[:, 0::32] = 1.0
    seen_k, seen_v = set(), set()
    p0 = orc.kivi_page_quantize(_f16(base_k).reshape(32, 128), _f16(base_v).reshape(32, 128))
    for t in range(0, 32, 7):
        for ch in range(1, 128, 13):
            k = base_k.copy(); k[t, ch] = 1.0 if t != 0 else 0.0
            p = orc.kivi_page_quantize(_f16(k).reshape(32, 128), _f16(base_v).reshape(32, 128))
            diff = np.nonzero(p[:2048] != p0[:2048])[0]
            assert len(diff) == 1
            seen_k.add((int(diff[0]), int(p[diff[0]] ^ p0[diff[0]])))
    assert len(seen_k) == len(range(0, 32, 7)) * len(range(1, 128, 13))


def test_kivi_page_roundtrip_error_bound():
    rng = np.random.default_rng(23)
    k = rng.standard_normal((32, 128)).astype(np.float32)
    k[:, [3, 40, 77, 100]] *= 8                          # outlier channels
    v = rng.standard_normal((32, 128)).astype(np.float32)
    kb, vb = _f16(k).reshape(32, 128), _f16(v).reshape(32, 128)
    page = orc.kivi_page_quantize(kb, vb)
    kd, vd = orc.kivi_page_dequant(page)
    kd = kd.view(np.float16).astype(np.float32)
    vd = vd.view(np.float16).astype(np.float32)
    kx, vx = kb.view(np.float16).astype(np.float32), vb.view(np.float16).astype(np.float32)
    # per-channel K groups over tokens; per-token V groups over 32 channels
    kstep = (kx.max(0) - kx.min(0)) / 15
    assert (np.abs(kd - kx) <= kstep[None, :] * 0.5 + np.abs(kx) * 2e-3 + 1e-3).all()
    vg = vx.reshape(32, 4, 32)
    vstep = (vg.max(2) - vg.min(2)) / 15
    err = np.abs(vd - vx).reshape(32, 4, 32)
    assert (err <= vstep[:, :, None] * 0.5 + np.abs(vg) * 2e-3 + 1e-3).all()


def test_kivi_page_constant_is_exact_and_params_land_in_place():
    k = np.full((32, 128), 1.5, np.float32)
    v = np.full((32, 128), -0.75, np.float32)
    page = orc.kivi_page_quantize(_f16(k).reshape(32, 128), _f16(v).reshape(32, 128))
    kd, vd = orc.kivi_page_dequant(page)
    assert (kd.view(np.float16) == 1.5).all() and (vd.view(np.float16) == -0.75).all()
    assert (page[:2048] == 0).all() and (page[2560:4608] == 0).all()
    kp = page[2048:2560].view(np.uint16).reshape(16, 2, 8)
    assert (kp[:, 0] == 0).all() and (kp[:, 1] == _f16(1.5)[0]).all()
    vp = page[4608:5120].view(np.uint16).reshape(16, 2, 8)
    assert (vp[:, 0] == 0).all() and (vp[:, 1] == _f16(-0.75)[0]).all()


# ---------------------------------------------------------------------------
# paged KIVI INT8 page format (KiviConfig.bits = 8)
# ---------------------------------------------------------------------------

def test_kivi_quant_group_levels_rne_and_int4_agreement():
    # 255 levels: 0..255 map to themselves; halfway cases round to even
    q, st, ze = orc.kivi_quant_group_levels(np.arange(256, dtype=np.float32), 255)
    assert list(q) == list(range(256)) and st == int(_f16(1.0)[0]) and ze == 0
    x = np.array([0.0, 1.0, 3.0, 5.0, 510.0], np.float32)          # scale 255/510 = 0.5
    q, _, _ = orc.kivi_quant_group_levels(x, 255)
    assert list(q) == [0, 0, 2, 2, 255]                             # 0.5 -> 0, 1.5 -> 2, 2.5 -> 2
    # 15 levels is the INT4 quantiser pinned above, bit for bit
    rng = np.random.default_rng(3)
    for n in (32, 7, 64):
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        a, b = orc.kivi_quant_group_levels(x, 15), orc.kivi_quant_group(x)
        assert np.array_equal(a[0], b[0]) and a[1:] == b[1:]


def _byte8(w0, w1):
    """The decode kernel's unpack of two code dwords: element order of the
    four masked fp16 pairs (low half first)."""
    out = []
    for w in (w0, w1):
        for sh in (0, 8):
            y = (int(w) >> sh) & 0x00FF00FF
            out += [y & 0xFF, y >> 16]
    return out


def test_kivi_int8_page_layout_matches_the_kernel_unpack():
    """For every lane chunk of a page, the kernel's unpack (two dwords per
    MFMA operand, 0x00FF00FF masks) yields the codes of the group quantiser
    (pinned above, computed here independently of the page layout) in the
    order the MFMA operands take them: K channels 8o .. 8o + 7 of token t for
    octet o = j + 4m; V token slots 0..7 of channel (4hh + m)*16 + u."""
    rng = np.random.default_rng(5)
    k = _f16((rng.standard_normal((32, 128)) * 2).astype(np.float32)).reshape(32, 128)
    v = _f16(rng.standard_normal((32, 128)).astype(np.float32)).reshape(32, 128)
    page = orc.kivi_page_quantize(k, v, 8)
    assert page.size == 9216
    kf, vf = k.view(np.float16).astype(np.float32), v.view(np.float16).astype(np.float32)
    kcode = np.stack([orc.kivi_quant_group_levels(kf[:, ch], 255)[0] for ch in range(128)])      # [ch][t]
    vcode = np.zeros((32, 128), np.int64)
    for t in range(32):
        for g in range(4):
            vcode[t, 32 * g:32 * g + 32] = orc.kivi_quant_group_levels(vf[t, 32 * g:32 * g + 32], 255)[0]
    dw = page[:8704].view(np.uint32)
    def v_token(r, s):
        return 4 * r + s if s < 4 else 16 + 4 * r + s - 4
    for c in range(128):
        tt, j, u = c // 64, (c % 64) // 16, c % 16
        t = tt * 16 + u
        for m in range(4):
            o = j + 4 * m
            got = _byte8(dw[c * 8 + 2 * m], dw[c * 8 + 2 * m + 1])
            assert got == [int(kcode[8 * o + e, t]) for e in range(8)], (c, m)
        hh, r = c // 64, (c % 64) // 16
        for m in range(4):
            d = (4 * hh + m) * 16 + u
            base = 4608 // 4 + c * 8 + 2 * m
            got = _byte8(dw[base], dw[base + 1])
            assert got == [int(vcode[v_token(r, s), d]) for s in range(8)], (c, m)


def test_kivi_int8_page_roundtrip_error_bound():
    rng = np.random.default_rng(23)
    k = rng.standard_normal((32, 128)).astype(np.float32)
    k[:, [3, 40, 77, 100]] *= 8
    v = rng.standard_normal((32, 128)).astype(np.float32)
    kb, vb = _f16(k).reshape(32, 128), _f16(v).reshape(32, 128)
    kd, vd = orc.kivi_page_dequant(orc.kivi_page_quantize(kb, vb, 8), 8)
    kd, vd = kd.view(np.float16).astype(np.float32), vd.view(np.float16).astype(np.float32)
    kx, vx = kb.view(np.float16).astype(np.float32), vb.view(np.float16).astype(np.float32)
    # x^ = fp16(n st + ze), st = fp16(range / 255), ze = fp16(min): the code
    # error is at most step / 2, the fp16 step adds up to 255 step 2^-11, the
    # fp16 zero |min| 2^-11 and the fp16 result |x| 2^-11
    u = 2.0 ** -11
    kmin, kstep = kx.min(0), (kx.max(0) - kx.min(0)) / 255
    kbound = kstep * (0.5 + 255 * u) + np.abs(kmin) * u
    assert (np.abs(kd - kx) <= kbound[None, :] + np.abs(kx) * u + 1e-6).all()
    vg = vx.reshape(32, 4, 32)
    vmin, vstep = vg.min(2), (vg.max(2) - vg.min(2)) / 255
    vbound = vstep * (0.5 + 255 * u) + np.abs(vmin) * u
    assert (np.abs(vd - vx).reshape(32, 4, 32) <= vbound[:, :, None] + np.abs(vg) * u + 1e-6).all()
    # 16 times finer than the INT4 page on the same data
    kd4, _ = orc.kivi_page_dequant(orc.kivi_page_quantize(kb, vb), 4)
    e4 = np.abs(kd4.view(np.float16).astype(np.float32) - kx).max()
    assert np.abs(kd - kx).max() < e4 / 8


def test_kivi_int8_page_constant_is_exact_and_params_land_in_place():
    k = np.full((32, 128), 1.5, np.float32)
    v = np.full((32, 128), -0.75, np.float32)
    page = orc.kivi_page_quantize(_f16(k).reshape(32, 128), _f16(v).reshape(32, 128), 8)
    kd, vd = orc.kivi_page_dequant(page, 8)
    assert (kd.view(np.float16) == 1.5).all() and (vd.view(np.float16) == -0.75).all()
    assert (page[:4096] == 0).all() and (page[4608:8704] == 0).all()
    kp = page[4096:4608].view(np.uint16).reshape(16, 2, 8)
    assert (kp[:, 0] == 0).all() and (kp[:, 1] == _f16(1.5)[0]).all()
    vp = page[8704:9216].view(np.uint16).reshape(16, 2, 8)
    assert (vp[:, 0] == 0).all() and (vp[:, 1] == _f16(-0.75)[0]).all()


def test_kivi_quantized_len():
    assert orc.kivi_quantized_len(0, 128) == 0
    assert orc.kivi_quantized_len(128, 128) == 0
    assert orc.kivi_quantized_len(159, 128) == 0
    assert orc.kivi_quantized_len(160, 128) == 32
    assert orc.kivi_quantized_len(4096, 128) == 3968
    for L in range(0, 600, 7):
        lq = orc.kivi_quantized_len(L, 128)
        assert lq % 32 == 0 and (L < 160 or 128 <= L - lq < 160)


def _kivi_small_case(seed, lens, n_kv=2, H=4):
    """fp16 pools (d 128, bs 16) with a page pool and a shuffled page table."""
    case = inputs.make_paged_case(seed, S=len(lens), H=H, n_kv=n_kv, D=128, BS=16, lens=lens,
                                  code=orc.F16)
    max_pages = max(1, max(lens) // 32 + 1)
    num_pages = len(lens) * max_pages + 2
    rng = np.random.default_rng(seed + 9)
    ptab = rng.permutation(num_pages)[: len(lens) * max_pages].astype(np.int32).reshape(len(lens), -1)
    return case, np.ascontiguousarray(ptab), num_pages


def _gather_tokens(pool, tables, s, t0, t1, kvh, BS=16):
    """[t1 - t0, 128] fp16 bits of tokens t0..t1-1 through the block table;
    zeros for a hole (numpy fancy indexing, independent of the oracle)."""
    pos = np.arange(t0, t1)
    phys = tables[s][pos // BS]
    out = pool[np.maximum(phys, 0), kvh, :, pos % BS].copy()
    out[phys < 0] = 0
    return out


def test_kivi_build_pages_equals_page_quantize_of_gathered_tokens():
    """orc_kivi_build_pages = orc_kivi_page_quantize (pinned above) applied to
    the tokens gathered through the block table, zeros for a block hole;
    page-table holes (negative or past the pool) are left untouched."""
    R = 128
    lens = [300, 161, 100, 223]
    case, ptab, num_pages = _kivi_small_case(31, lens)
    case.tables[0, 3] = -1                 # tokens 48..63: page 1 of sequence 0
    ptab[0, 2] = -1                        # page holes: negative and past the pool
    ptab[0, 4] = num_pages
    n_kv = 2
    pages = np.full((num_pages, n_kv, orc.KIVI_PAGE_BYTES), 0xA5, np.uint8)
    orc.kivi_build_pages(case.k_cache, case.v_cache, case.tables, case.seq_lens, R, pages, ptab)
    want = np.full_like(pages, 0xA5)
    built = 0
    for s, L in enumerate(lens):
        for p in range(orc.kivi_quantized_len(L, R) // 32):
            pid = int(ptab[s, p])
            if pid < 0 or pid >= num_pages:
                continue
            for h in range(n_kv):
                kt = _gather_tokens(case.k_cache, case.tables, s, 32 * p, 32 * p + 32, h)
                vt = _gather_tokens(case.v_cache, case.tables, s, 32 * p, 32 * p + 32, h)
                want[pid, h] = orc.kivi_page_quantize(np.ascontiguousarray(kt), np.ascontiguousarray(vt))
                built += 1
    assert built == (5 - 2 + 1 + 0 + 2) * n_kv     # Lq: 160, 32, 0, 64 tokens
    assert np.array_equal(pages, want)


def _kivi_as_paged_pool(case, pages, ptab, num_pages, R, bits=4):
    """The pool a KIVI cache stands for: tokens below Lq dequantised from
    their page (a page hole: both of its blocks are table holes), the rest
    copied from the fp16 pool through the block table.  Each sequence gets
    contiguous blocks of a fresh pool."""
    S, H, D = case.q.shape
    n_kv, BS = case.k_cache.shape[1], 16
    nblk = [(int(L) + BS - 1) // BS for L in case.seq_lens]
    kp = np.zeros((sum(nblk) + 1, n_kv, D, BS), np.uint16)
    vp = np.zeros_like(kp)
    tables = np.full((S, max(nblk)), -1, np.int32)
    nxt = 0
    for s, L in enumerate(case.seq_lens):
        L = int(L)
        Lq = orc.kivi_quantized_len(L, R)
        for b in range(nblk[s]):
            t0, t1 = b * BS, min(L, b * BS + BS)
            if t0 < Lq:
                pid = int(ptab[s, t0 // 32])
                if pid < 0 or pid >= num_pages:
                    continue
                for h in range(n_kv):
                    kd, vd = orc.kivi_page_dequant(np.ascontiguousarray(pages[pid, h]), bits)
                    o = t0 % 32
                    kp[nxt, h] = kd[o:o + BS].T
                    vp[nxt, h] = vd[o:o + BS].T
            else:
                if case.tables[s, b] < 0:
                    continue
                for h in range(n_kv):
                    kp[nxt, h, :, : t1 - t0] = _gather_tokens(case.k_cache, case.tables, s, t0, t1, h).T
                    vp[nxt, h, :, : t1 - t0] = _gather_tokens(case.v_cache, case.tables, s, t0, t1, h).T
            tables[s, b] = nxt
            nxt += 1
    return kp, vp, tables


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gqa_map", [orc.MODULO, orc.GROUPED])
def test_kivi_attention_equals_paged_attention_on_dequantised_prefix(gqa_map, bits):
    """orc_kivi_paged_attention = orc_paged_attention (pinned above) over the
    pool it stands for: pages dequantised by orc_kivi_page_dequant below Lq,
    the fp16 window above; page-table holes and block-table holes in the
    window drop their tokens, a block hole inside a built page does not (the
    page holds its quantised zeros)."""
    R = 128
    lens = [300, 161, 100, 223]
    case, ptab, num_pages = _kivi_small_case(32, lens)
    case.tables[0, 3] = -1                 # inside page 1 of sequence 0
    case.tables[0, 12] = -1                # in the window of sequence 0 (Lq = 160)
    case.tables[3, 9] = -1                 # in the window of sequence 3 (Lq = 64)
    ptab[0, 2] = -1
    ptab[3, 1] = num_pages                 # past the pool: a hole too
    pages = np.zeros((num_pages, 2, orc.kivi_page_bytes(bits)), np.uint8)
    orc.kivi_build_pages(case.k_cache, case.v_cache, case.tables, case.seq_lens, R, pages, ptab, bits)
    got = orc.kivi_paged_attention(case.q, orc.F16, pages, ptab, case.k_cache, case.v_cache,
                                   case.tables, case.seq_lens, 2, R, case.scale, gqa_map, bits)
    kp, vp, t2 = _kivi_as_paged_pool(case, pages, ptab, num_pages, R, bits)
    want = orc.paged_attention(case.q, orc.F16, kp, vp, orc.F16, t2, case.seq_lens, 2, case.scale,
                               gqa_map)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-12)
    # the holes matter: without them the result changes
    full = orc.kivi_paged_attention(case.q, orc.F16, pages, np.where(ptab >= num_pages, 0, np.abs(ptab)).astype(np.int32),
                                    case.k_cache, case.v_cache, case.tables, case.seq_lens, 2, R, case.scale,
                                    gqa_map, bits)
    assert np.abs(full[0] - got[0]).max() > 1e-3 and np.abs(full[3] - got[3]).max() > 1e-3


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gqa_map", [orc.MODULO, orc.GROUPED])
def test_cpu_baseline_kivi_f32_matches_oracle(gqa_map, bits):
    """The CPU baseline's paged KIVI decode (fp32, threads) against the fp64
    oracle, holes of both kinds included: within an fp16 output ulp and the
    fp32 sums' rounding."""
    R = 128
    case, ptab, num_pages = _kivi_small_case(33, [300, 161, 100, 223])
    case.tables[0, 12] = -1
    ptab[0, 2] = -1
    ptab[3, 1] = num_pages
    pages = np.zeros((num_pages, 2, orc.kivi_page_bytes(bits)), np.uint8)
    orc.kivi_build_pages(case.k_cache, case.v_cache, case.tables, case.seq_lens, R, pages, ptab, bits)
    want = orc.kivi_paged_attention(case.q, orc.F16, pages, ptab, case.k_cache, case.v_cache,
                                    case.tables, case.seq_lens, 2, R, case.scale, gqa_map, bits)
    got = orc.kivi_paged_attention_f32(case.q, pages, ptab, case.k_cache, case.v_cache, case.tables,
                                       case.seq_lens, 2, R, case.scale, gqa_map, bits, threads=3)
    got = got.view(np.float16).astype(np.float64)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-5 + np.abs(want).max() * 2.0 ** -11)
    assert np.abs(want).max() > 0.1


@pytest.mark.parametrize("style,bits", [(0, 4), (1, 4), (0, 8), (1, 8)])
def test_kivi_pre_rope_attention_is_attention_on_the_rotated_pool(style, bits):
    """Keys held before RoPE (KiviConfig.pre_rope_keys): the oracle's KIVI
    attention with the tables equals orc_paged_attention (pinned above) on
    the pool the cache stands for (dequantised pages below Lq, the window
    above) in fp32, each valid token's key rotated at its position by
    orc_rope_reshape_and_cache (pinned by its own tests).  The tables stop
    at 280: sequence 0's later tokens stay unrotated.  Holes in the page
    table and in the window drop their tokens."""
    R = 128
    lens = [300, 161, 100, 223]
    case, ptab, num_pages = _kivi_small_case(34, lens)
    case.tables[0, 12] = -1
    ptab[3, 1] = -1
    pages = np.zeros((num_pages, 2, orc.kivi_page_bytes(bits)), np.uint8)
    orc.kivi_build_pages(case.k_cache, case.v_cache, case.tables, case.seq_lens, R, pages, ptab, bits)
    cos_t, sin_t = rope_tables(280, 128)
    got = orc.kivi_paged_attention(case.q, orc.F16, pages, ptab, case.k_cache, case.v_cache, case.tables,
                                   case.seq_lens, 2, R, case.scale, orc.GROUPED, bits, pre_rope=(cos_t, sin_t, style))
    kp, vp, t2 = _kivi_as_paged_pool(case, pages, ptab, num_pages, R, bits)
    f32 = lambda a: orc.bits_to_f32(a, orc.F16).astype(np.float32).view(np.uint32)
    kp32, vp32 = np.ascontiguousarray(f32(kp)), np.ascontiguousarray(f32(vp))
    rows_k, rows_v, slots, pos = [], [], [], []
    for si, L in enumerate(case.seq_lens):
        for t in range(int(L)):
            blk = int(t2[si, t // 16])
            if blk < 0:
                continue
            rows_k.append(kp32[blk, :, :, t % 16])
            rows_v.append(vp32[blk, :, :, t % 16])
            slots.append(blk * 16 + t % 16)
            pos.append(t)
    rk, rv = np.ascontiguousarray(np.stack(rows_k)), np.ascontiguousarray(np.stack(rows_v))
    orc.rope_reshape_and_cache(None, None, rk, rv, kp32, vp32, np.array(slots, np.int32), np.array(pos, np.int32),
                               cos_t, sin_t, orc.F32, style)
    want = orc.paged_attention(case.q, orc.F16, kp32, vp32, orc.F32, t2, case.seq_lens, 2, case.scale,
                               orc.GROUPED)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-5)
    plain = orc.kivi_paged_attention(case.q, orc.F16, pages, ptab, case.k_cache, case.v_cache, case.tables,
                                     case.seq_lens, 2, R, case.scale, orc.GROUPED, bits)
    assert np.abs(plain - got).max() > 1e-2


def test_kivi_attention_without_pages_is_paged_attention_with_holes():
    """R >= L: no token is quantised, so KIVI attention is paged attention on
    the fp16 pool, holes skipped in both."""
    lens = [300, 161, 100, 1]
    case, ptab, num_pages = _kivi_small_case(33, lens)
    case.tables[0, 5] = -1
    case.tables[2, 0] = -1
    pages = np.zeros((num_pages, 2, orc.KIVI_PAGE_BYTES), np.uint8)
    got = orc.kivi_paged_attention(case.q, orc.F16, pages, ptab, case.k_cache, case.v_cache,
                                   case.tables, case.seq_lens, 2, 512, case.scale, orc.GROUPED)
    want = orc.paged_attention(case.q, orc.F16, case.k_cache, case.v_cache, orc.F16, case.tables,
                               case.seq_lens, 2, case.scale, orc.GROUPED)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-12)
    np.testing.assert_allclose(got, numpy_attention(case, orc.GROUPED), rtol=0, atol=1e-12)


def test_kivi_attention_all_holes_gives_zeros():
    lens = [200, 40]
    case, ptab, num_pages = _kivi_small_case(34, lens)
    ptab[0, :] = -1                        # both pages of sequence 0 (Lq = 64)
    case.tables[0, 4:] = -1                # and its whole window
    case.tables[1, :] = -1
    pages = np.zeros((num_pages, 2, orc.KIVI_PAGE_BYTES), np.uint8)
    got = orc.kivi_paged_attention(case.q, orc.F16, pages, ptab, case.k_cache, case.v_cache,
                                   case.tables, case.seq_lens, 2, 128, case.scale, orc.GROUPED)
    assert (got == 0).all()


@pytest.mark.parametrize("code", [orc.F16, orc.BF16])
def test_reshape_and_cache_fp8_is_scatter_of_e4m3_codes(code):
    """orc_reshape_and_cache_fp8 = torch's float8_e4m3fn encode of
    x * fp32(1 / scale) (an independent RNE implementation) scattered by the
    slot map with numpy indexing; slot < 0 skipped, other slots untouched."""
    rng = np.random.default_rng(35)
    T, n_kv, D, BS, N = 37, 4, 64, 16, 9
    xk = rng.standard_normal((T, n_kv, D), dtype=np.float32)
    xv = rng.standard_normal((T, n_kv, D), dtype=np.float32) * 3
    kb, vb = inputs.encode(xk, code), inputs.encode(xv, code)
    kf, vf = orc.bits_to_f32(kb, code), orc.bits_to_f32(vb, code)
    ks, vs = float(np.abs(kf).max()) / 448, float(np.abs(vf).max()) / 448
    slots = rng.permutation(N * BS)[:T].astype(np.int32)
    slots[[4, 20]] = -1
    kc = rng.integers(0, 256, (N, n_kv, D, BS), dtype=np.uint8)
    vc = rng.integers(0, 256, (N, n_kv, D, BS), dtype=np.uint8)
    want_k, want_v = kc.copy(), vc.copy()
    orc.reshape_and_cache_fp8(kb, vb, code, kc, vc, slots, ks, vs)

    def e4m3(x, s):
        mul = np.float32(1.0) / np.float32(s)
        return torch.from_numpy(x * mul).to(torch.float8_e4m3fn).view(torch.uint8).numpy()

    ck, cv = e4m3(kf, ks), e4m3(vf, vs)
    for t, sl in enumerate(slots):
        if sl < 0:
            continue
        want_k[sl // BS, :, :, sl % BS] = ck[t]
        want_v[sl // BS, :, :, sl % BS] = cv[t]
    assert np.array_equal(kc, want_k) and np.array_equal(vc, want_v)


# ---------------------------------------------------------------------------
# block management (copy_blocks / swap_blocks)
# ---------------------------------------------------------------------------

def _pools(rng, n, shape, dtype):
    k = rng.integers(0, 256, size=(n,) + shape + (np.dtype(dtype).itemsize,), dtype=np.uint8)
    v = rng.integers(0, 256, size=k.shape, dtype=np.uint8)
    return k.view(dtype).reshape((n,) + shape), v.view(dtype).reshape((n,) + shape)


@pytest.mark.parametrize("dtype", [np.float16, np.float32, np.uint8])
def test_copy_blocks_oracle_matches_fancy_indexing(dtype):
    """orc_copy_blocks against numpy's pool[dst] = pool[src] for distinct
    destinations that are not sources; K and V move independently, other
    blocks keep their bytes, out-of-range pairs are skipped."""
    rng = np.random.default_rng(21)
    N = 24
    k, v = _pools(rng, N, (2, 8, 16), dtype)
    perm = rng.permutation(N)
    src, dst = perm[:8], perm[8:16]
    mapping = np.stack([src, dst], 1).astype(np.int32)
    bad = np.array([[-1, 3], [2, N], [N + 5, 0]], np.int32)
    full = np.concatenate([mapping, bad]).copy()
    ek, ev = k.copy(), v.copy()
    ek[dst] = k[src]
    ev[dst] = v[src]
    orc.copy_blocks(k, v, full)
    assert np.array_equal(k.view(np.uint8), ek.view(np.uint8))
    assert np.array_equal(v.view(np.uint8), ev.view(np.uint8))


def test_copy_blocks_oracle_identity_is_a_no_op():
    rng = np.random.default_rng(22)
    k, v = _pools(rng, 6, (4, 4), np.float16)
    k0, v0 = k.copy(), v.copy()
    orc.copy_blocks(k, v, np.array([[i, i] for i in range(6)], np.int32))
    assert np.array_equal(k.view(np.uint16), k0.view(np.uint16))
    assert np.array_equal(v.view(np.uint16), v0.view(np.uint16))


def test_swap_blocks_oracle_round_trip():
    """Out to the host buffer (direction 0) and back (direction 1) restores
    the evicted blocks; each direction matches numpy indexing."""
    rng = np.random.default_rng(23)
    dev_pool, _ = _pools(rng, 20, (8, 16), np.float16)
    host = np.zeros((10,) + dev_pool.shape[1:], np.float16)
    src = np.array([3, 17, 0, 9], np.int32)
    slots = np.array([7, 0, 2, 9], np.int32)
    out_map = np.stack([src, slots], 1).astype(np.int32).copy()
    orc.swap_blocks(dev_pool, host, out_map, 0)
    assert np.array_equal(host[slots].view(np.uint16), dev_pool[src].view(np.uint16))
    saved = dev_pool[src].copy()
    dev_pool[src] = 0
    back = np.stack([slots, src], 1).astype(np.int32).copy()
    orc.swap_blocks(dev_pool, host, back, 1)
    assert np.array_equal(dev_pool[src].view(np.uint16), saved.view(np.uint16))
    # ids outside either pool skip the pair
    before = host.copy()
    orc.swap_blocks(dev_pool, host, np.array([[20, 0], [0, 10], [-1, 1]], np.int32), 0)
    assert np.array_equal(host.view(np.uint16), before.view(np.uint16))


# ---------------------------------------------------------------------------
# RoPE + reshape_and_cache
# ---------------------------------------------------------------------------

def rope_tables(max_pos, D, base=10000.0):
    """cuda_model.cpp:269-295: theta = pos / base^(2i/D), fp32 tables [max_pos, D/2]."""
    i = np.arange(D // 2, dtype=np.float32)
    pos = np.arange(max_pos, dtype=np.float32)[:, None]
    theta = pos / np.power(np.float32(base), np.float32(2.0) * i / np.float32(D))
    return np.cos(theta).astype(np.float32), np.sin(theta).astype(np.float32)


def _pair_mag(x, style):
    """|a| + |b| of each element's pair: the scale of the fp32 rounding error."""
    D = x.shape[-1]
    half = D // 2
    i = np.arange(half)
    d0, d1 = (2 * i, 2 * i + 1) if style == 0 else (i, i + half)
    m = np.zeros(x.shape, np.float64)
    pm = np.abs(x[..., d0]).astype(np.float64) + np.abs(x[..., d1])
    m[..., d0] = pm
    m[..., d1] = pm
    return m


def _rope_np(x, pos, cos_t, sin_t, style):
    """float64 rotation of rows x [..., D] at positions pos (one per leading row)."""
    D = x.shape[-1]
    half = D // 2
    i = np.arange(half)
    d0, d1 = (2 * i, 2 * i + 1) if style == 0 else (i, i + half)
    c = cos_t[pos].astype(np.float64)[..., None, :] if x.ndim == 3 else cos_t[pos].astype(np.float64)
    s = sin_t[pos].astype(np.float64)[..., None, :] if x.ndim == 3 else sin_t[pos].astype(np.float64)
    a, b = x[..., d0].astype(np.float64), x[..., d1].astype(np.float64)
    out = x.astype(np.float64).copy()
    out[..., d0] = a * c - b * s
    out[..., d1] = a * s + b * c
    return out


def _rope_case(seed, T, H, n_kv, D, BS, N, code, max_pos=4096):
    rng = np.random.default_rng(seed)
    q = inputs.encode(rng.standard_normal((T, H, D), dtype=np.float32), code)
    key = inputs.encode(rng.standard_normal((T, n_kv, D), dtype=np.float32), code)
    val = inputs.encode(rng.standard_normal((T, n_kv, D), dtype=np.float32), code)
    slots = rng.choice(N * BS, size=T, replace=False).astype(np.int32)
    pos = rng.integers(0, max_pos, size=T).astype(np.int32)
    kc = inputs.encode(np.zeros((N, n_kv, D, BS), np.float32), code)
    vc = inputs.encode(np.zeros((N, n_kv, D, BS), np.float32), code)
    return q, key, val, slots, pos, kc, vc


@pytest.mark.parametrize("style", [0, 1])
@pytest.mark.parametrize("code", [orc.F16, orc.BF16, orc.F32])
def test_rope_oracle_matches_float64_rotation(style, code):
    """Each style's pairing against a float64 rotation with the same fp32
    tables: within one unit in the last place of the dtype (a wrong pairing
    or a sign error is off by O(1)); values pass through the pool unchanged."""
    T, H, n_kv, D, BS, N = 9, 4, 2, 64, 16, 8
    q, key, val, slots, pos, kc, vc = _rope_case(40 + style, T, H, n_kv, D, BS, N, code)
    cos_t, sin_t = rope_tables(4096, D)
    q_out = np.zeros_like(q)
    orc.rope_reshape_and_cache(q, q_out, key, val, kc, vc, slots, pos, cos_t, sin_t, code, style)
    qf = orc.bits_to_f32(q, code) if code != orc.F32 else q
    kf = orc.bits_to_f32(key, code) if code != orc.F32 else key
    want_q = _rope_np(qf, pos, cos_t, sin_t, style)
    want_k = _rope_np(kf, pos, cos_t, sin_t, style)
    got_q = orc.bits_to_f32(q_out, code) if code != orc.F32 else q_out
    # one unit in the last place of the dtype at the result, plus the fp32
    # rounding of the two products (relative to the pair's magnitude)
    ulp = {orc.F16: 2.0 ** -10, orc.BF16: 2.0 ** -7, orc.F32: 2.0 ** -23}[code]
    tol = ulp * np.maximum(np.abs(want_q), 2.0 ** -14) + 2.0 ** -22 * _pair_mag(qf, style)
    assert np.all(np.abs(got_q - want_q) <= tol)
    blk, off = slots // BS, slots % BS
    got_k = np.stack([(orc.bits_to_f32(kc, code) if code != orc.F32 else kc)[blk[t], :, :, off[t]]
                      for t in range(T)])
    assert np.all(np.abs(got_k - want_k) <= ulp * np.maximum(np.abs(want_k), 2.0 ** -14)
                  + 2.0 ** -22 * _pair_mag(kf, style))
    got_v = np.stack([vc[blk[t], :, :, off[t]] for t in range(T)])
    assert np.array_equal(got_v, val)


def test_rope_oracle_position_zero_is_identity_and_skips():
    """Position 0 (cos 1, sin 0) leaves q and k as they are, so the pools
    equal a plain reshape_and_cache; slot -1 writes no pool; a position past
    the tables writes nothing."""
    T, H, n_kv, D, BS, N = 6, 3, 2, 32, 16, 4
    q, key, val, slots, pos, kc, vc = _rope_case(44, T, H, n_kv, D, BS, N, orc.F16)
    cos_t, sin_t = rope_tables(64, D)
    pos[:] = 0
    slots[2] = -1
    pos[4] = 64
    q_out = np.zeros_like(q)
    orc.rope_reshape_and_cache(q, q_out, key, val, kc, vc, slots, pos, cos_t, sin_t, orc.F16, 0)
    keep = np.ones(T, bool)
    keep[4] = False
    assert np.array_equal(q_out[keep], q[keep]) and not q_out[4].any()
    ek, ev = np.zeros_like(kc), np.zeros_like(vc)
    s2 = slots.copy()
    s2[4] = -1
    orc.reshape_and_cache(key, val, ek, ev, s2)
    assert np.array_equal(kc, ek) and np.array_equal(vc, ev)


def test_rope_oracle_preserves_pair_norms_with_reference_tables():
    """Rotation keeps |(a, b)| of every pair (fp32 data, reference tables at
    positions up to 4095)."""
    T, H, n_kv, D, BS, N = 16, 2, 1, 128, 16, 2
    q, key, val, slots, pos, kc, vc = _rope_case(45, T, H, n_kv, D, BS, N, orc.F32)
    cos_t, sin_t = rope_tables(4096, D)
    for style in (0, 1):
        q_out = np.zeros_like(q)
        orc.rope_reshape_and_cache(q, q_out, key, val, kc.copy(), vc.copy(), slots, pos, cos_t, sin_t,
                                   orc.F32, style)
        i = np.arange(D // 2)
        d0, d1 = (2 * i, 2 * i + 1) if style == 0 else (i, i + D // 2)
        n_in = np.hypot(q[..., d0], q[..., d1])
        n_out = np.hypot(q_out[..., d0], q_out[..., d1])
        assert np.allclose(n_in, n_out, rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------------------
# VQ codec
# ---------------------------------------------------------------------------

def _f16(x):
    return orc.f32_to_f16_bits(np.asarray(x, np.float32))


def test_vq_oracle_reference_known_answers():
    """test_vq_kernels.cpp:96-204: exact copies encode to their own entry and
    decode back; perturbations of +-1 around entries 1000 apart pick the
    nearest; decode of synthetic indices reads those rows."""
    book = _f16([[c * 10 + d for d in range(8)] for c in range(4)])
    want = np.array([(t * 2 + h) % 4 for t in range(4) for h in range(2)], np.uint16)
    kv = book[want]
    idx = orc.vq_encode(kv, book)
    assert np.array_equal(idx, want)
    out = np.zeros_like(kv)
    orc.vq_decode(out, book, idx)
    assert np.array_equal(out, kv)
    book2 = _f16([[0] * 4, [1000] * 4, [2000] * 4])
    kv2 = _f16([[0.5, -0.5, 0.2, -0.2], [1001, 999, 1000.5, 999.5], [1999, 2001, 1999.5, 2000.5]])
    assert np.array_equal(orc.vq_encode(kv2, book2), np.array([0, 1, 2], np.uint16))
    book3 = _f16([[100 * c + d for d in range(4)] for c in range(5)])
    idx3 = np.array([4, 0, 2, 3], np.uint16)
    out3 = np.zeros((4, 4), np.uint16)
    orc.vq_decode(out3, book3, idx3)
    assert np.array_equal(out3, book3[idx3])


def test_vq_oracle_nearest_ties_and_nan():
    """Against float64 brute force: the chosen entry's distance is the
    minimum (up to fp32 rounding); among equal rows the lowest index wins;
    a vector holding NaN gets index 0."""
    rng = np.random.default_rng(50)
    K, D, n = 64, 32, 200
    book = _f16(rng.standard_normal((K, D)))
    book[40] = book[7]                                   # a duplicated entry: 7 must win
    kv = _f16(rng.standard_normal((n, D)))
    kv[5] = book[7]
    idx = orc.vq_encode(kv, book)
    bf, xf = orc.bits_to_f32(book, orc.F16).astype(np.float64), orc.bits_to_f32(kv, orc.F16).astype(np.float64)
    d64 = ((xf[:, None, :] - bf[None, :, :]) ** 2).sum(-1)
    chosen = d64[np.arange(n), idx.astype(int)]
    assert np.all(chosen <= d64.min(1) * (1 + 1e-5) + 1e-6)
    assert idx[5] == 7 and not np.any(idx == 40)
    kv[9, 3] = 0x7E00                                    # NaN
    assert orc.vq_encode(kv, book)[9] == 0


def test_vq_kmeans_oracle_exact_means_order_independent_and_empty_clusters():
    """One Lloyd step on three well-separated groups: each centroid is its
    members' mean (to one fp16 ulp); the book does not depend on the order
    of the samples (exact sums); an entry that attracts no sample keeps its
    value."""
    rng = np.random.default_rng(51)
    D = 16
    centres = np.array([0.0, 50.0, -80.0])
    data = np.concatenate([c + rng.standard_normal((30, D)) for c in centres]).astype(np.float32)
    bits = _f16(data)
    book0 = _f16(np.stack([np.full(D, c + 0.3) for c in centres] + [np.full(D, 1e4)]))
    book = book0.copy()
    orc.vq_kmeans(bits, book, 1)
    xf = orc.bits_to_f32(bits, orc.F16).astype(np.float64)
    for g in range(3):
        want = xf[30 * g:30 * (g + 1)].mean(0)
        got = orc.bits_to_f32(book[g], orc.F16)
        assert np.all(np.abs(got - want) <= 2.0 ** -10 * np.maximum(np.abs(want), 2.0 ** -14))
    assert np.array_equal(book[3], book0[3])
    perm = rng.permutation(len(bits))
    book_p = book0.copy()
    orc.vq_kmeans(bits[perm].copy(), book_p, 1)
    assert np.array_equal(book, book_p)
    book3 = book0.copy()
    orc.vq_kmeans(bits, book3, 3)
    assert np.array_equal(book3[:3], book[:3])          # converged after one step


# ---------------------------------------------------------------------------
# norms and gated activations
# ---------------------------------------------------------------------------

def test_norm_act_oracle_reference_known_answers():
    """test_vllm_kernels.cpp:128-253: RMSNorm of a 2 x 8 ramp against the
    double reference (1e-4), uniform input with eps 0 gives 1, silu_and_mul
    of ramps against x / (1 + exp(-x)) * up (1e-5), up = 0 gives 0."""
    T, H = 2, 8
    x = (0.1 * (np.arange(T * H) + 1)).astype(np.float32).reshape(T, H)
    w = (1.0 - 0.05 * np.arange(H)).astype(np.float32)
    got = orc.rms_norm(x, w, 1e-5, orc.F32)
    xd = x.astype(np.float64)
    want = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + 1e-5) * w
    assert np.allclose(got, want, atol=1e-4, rtol=0)
    u = np.full((1, 32), 2.5, np.float32)
    assert np.allclose(orc.rms_norm(u, np.ones(32, np.float32), 0.0, orc.F32), 1.0, atol=1e-4)
    g = (-1.0 + 0.07 * np.arange(64)).astype(np.float32).reshape(4, 16)
    up = (0.25 + 0.03 * np.arange(64)).astype(np.float32).reshape(4, 16)
    got = orc.act_and_mul(g, up, 0, orc.F32)
    gd = g.astype(np.float64)
    assert np.allclose(got, gd / (1 + np.exp(-gd)) * up, atol=1e-5, rtol=0)
    g2 = (np.arange(128) - 64).astype(np.float32).reshape(2, 64)
    assert not np.any(orc.act_and_mul(g2, np.zeros_like(g2), 0, orc.F32))


def test_fused_add_rms_norm_and_layer_norm_oracle_closed_forms():
    """fused_add_rms_norm = residual update (res + x rounded) followed by the
    mean square of the unrounded sums applied to the rounded residual;
    layer_norm against float64 mean / variance, and a constant row gives the
    bias."""
    rng = np.random.default_rng(70)
    T, H = 5, 96
    code = orc.BF16
    x = inputs.encode(rng.standard_normal((T, H), dtype=np.float32), code)
    res = inputs.encode(rng.standard_normal((T, H), dtype=np.float32), code)
    w = inputs.encode(1 + 0.1 * rng.standard_normal(H, dtype=np.float32), code)
    r = res.copy()
    out = orc.rms_norm(x, w, 1e-6, code, residual=r)
    s32 = orc.bits_to_f32(res, code) + orc.bits_to_f32(x, code)
    assert np.array_equal(r, orc.f32_to_bf16_bits(s32))
    inv = 1.0 / np.sqrt((s32.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6)
    want = orc.bits_to_f32(r, code) * inv * orc.bits_to_f32(w, code)
    got = orc.bits_to_f32(out, code)
    assert np.all(np.abs(got - want) <= 2.0 ** -7 * np.abs(want) + 1e-6)
    xf = rng.standard_normal((T, H)).astype(np.float32)
    wf = rng.standard_normal(H).astype(np.float32)
    bf = rng.standard_normal(H).astype(np.float32)
    got = orc.layer_norm(xf, wf, bf, 1e-5, orc.F32)
    xd = xf.astype(np.float64)
    want = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-5) * wf + bf
    assert np.allclose(got, want, atol=1e-5, rtol=1e-5)
    const = np.full((2, H), 3.0, np.float32)
    assert np.allclose(orc.layer_norm(const, wf, bf, 1e-5, orc.F32), bf, atol=1e-6)


def test_gelu_oracle_matches_float64_formulas():
    import math
    g = np.linspace(-6, 6, 241).astype(np.float32).reshape(1, -1)
    up = np.ones_like(g)
    got = orc.act_and_mul(g, up, 1, orc.F32)
    want = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in g.ravel().astype(np.float64)])
    assert np.allclose(got.ravel(), want, atol=1e-6, rtol=1e-5)
    got = orc.act_and_mul(g, up, 2, orc.F32)
    gd = g.ravel().astype(np.float64)
    want = 0.5 * gd * (1 + np.tanh(0.79788456 * (gd + 0.044715 * gd ** 3)))
    assert np.allclose(got.ravel(), want, atol=1e-6, rtol=1e-5)
