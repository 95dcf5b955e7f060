"""Bit-exact parity of the gfx950 KV-cache writes against the oracle."""
import numpy as np
import pytest
import torch

import inputs
import oracle_lib as orc
import tl_attn as tla
from gpu_util import dev, host_bits

pytestmark = pytest.mark.gpu


def _slots_case(seed, T, n_kv, D, BS, N, code):
    rng = np.random.default_rng(seed)
    slots = rng.choice(N * BS, size=T, replace=False).astype(np.int32)
    slots[::5] = -1                                     # padded tokens
    key = inputs.encode(rng.standard_normal((T, n_kv, D), dtype=np.float32), code)
    val = inputs.encode(rng.standard_normal((T, n_kv, D), dtype=np.float32), code)
    kc = inputs.encode(rng.standard_normal((N, n_kv, D, BS), dtype=np.float32), code)
    vc = inputs.encode(rng.standard_normal((N, n_kv, D, BS), dtype=np.float32), code)
    return key, val, kc, vc, slots


@pytest.mark.parametrize("code", [orc.F16, orc.BF16, orc.F32])
@pytest.mark.parametrize("T,n_kv,D,BS", [(64, 8, 128, 16), (37, 2, 64, 32), (5, 3, 256, 16),
                                         (200, 8, 128, 16)])
def test_reshape_and_cache_bit_exact(code, T, n_kv, D, BS):
    N = 64
    key, val, kc, vc, slots = _slots_case(T * 7 + D, T, n_kv, D, BS, N, code)
    kd, vd, kcd, vcd = dev(key, code), dev(val, code), dev(kc, code), dev(vc, code)
    print(f"case reshape code={code} T={T} D={D} BS={BS}", flush=True)
    tla.reshape_and_cache_split(kd, vd, kcd, vcd, dev(slots))
    torch.cuda.synchronize()
    orc.reshape_and_cache(key, val, kc, vc, slots)
    assert np.array_equal(host_bits(kcd), kc)
    assert np.array_equal(host_bits(vcd), vc)


@pytest.mark.parametrize("code", [orc.F16, orc.BF16, orc.F32])
@pytest.mark.parametrize("T,n_kv,D,BS", [(64, 8, 128, 16), (33, 2, 64, 32), (256, 4, 128, 16), (300, 2, 128, 16)])
def test_reshape_and_cache_decode_append_bit_exact(code, T, n_kv, D, BS):
    """One token per block (a decode step's append: the whole-row path for
    up to 256 tokens, element stores past that), over a pool of random
    bytes that every other slot must keep; a few tokens share a block or
    are padded."""
    N = 2 * T + 8
    rng = np.random.default_rng(T + D)
    blocks = rng.permutation(N)[:T]
    slots = (blocks * BS + rng.integers(0, BS, size=T)).astype(np.int32)
    slots[7] = slots[3] - slots[3] % BS + (slots[3] % BS + 1) % BS   # token 7 shares token 3's block
    slots[11] = -1
    key = inputs.encode(rng.standard_normal((T, n_kv, D), dtype=np.float32), code)
    val = inputs.encode(rng.standard_normal((T, n_kv, D), dtype=np.float32), code)
    kc = inputs.encode(rng.standard_normal((N, n_kv, D, BS), dtype=np.float32), code)
    vc = inputs.encode(rng.standard_normal((N, n_kv, D, BS), dtype=np.float32), code)
    kd, vd, kcd, vcd = dev(key, code), dev(val, code), dev(kc, code), dev(vc, code)
    print(f"case reshape append code={code} T={T} D={D} BS={BS}", flush=True)
    tla.reshape_and_cache_split(kd, vd, kcd, vcd, dev(slots))
    torch.cuda.synchronize()
    orc.reshape_and_cache(key, val, kc, vc, slots)
    assert np.array_equal(host_bits(kcd), kc)
    assert np.array_equal(host_bits(vcd), vc)


def test_reshape_and_cache_reference_layout_and_out_of_pool_slots():
    """kv_cache [2N, n_kv, D, BS] = K pool then V pool (cache_kernels.cu:27-33);
    slots past the pool are skipped instead of written out of bounds."""
    code, T, n_kv, D, BS, N = orc.F16, 16, 2, 128, 16, 8
    key, val, kc, vc, slots = _slots_case(5, T, n_kv, D, BS, N, code)
    slots[3] = N * BS + 5
    kv = np.concatenate([kc, vc])
    kvd = dev(kv, code)
    tla.reshape_and_cache(dev(key, code), dev(val, code), kvd, dev(slots))
    torch.cuda.synchronize()
    slots_ok = slots.copy()
    slots_ok[3] = -1
    orc.reshape_and_cache(key, val, kc, vc, slots_ok)
    assert np.array_equal(host_bits(kvd), np.concatenate([kc, vc]))


@pytest.mark.parametrize("code", [orc.F16, orc.BF16])
def test_reshape_and_cache_fp8_bit_exact(code):
    T, n_kv, D, BS, N = 96, 8, 128, 16, 32
    key, val, _, _, slots = _slots_case(9, T, n_kv, D, BS, N, code)
    k8 = np.random.default_rng(1).integers(0, 255, (N, n_kv, D, BS), dtype=np.uint8)
    v8 = k8[::-1].copy()
    kd8, vd8 = torch.from_numpy(k8.copy()).cuda(), torch.from_numpy(v8.copy()).cuda()
    ks, vs = 3.1 / 448, 0.02
    print(f"case reshape fp8 code={code}", flush=True)
    tla.reshape_and_cache_fp8(dev(key, code), dev(val, code), kd8, vd8, dev(slots), ks, vs)
    torch.cuda.synchronize()
    orc.reshape_and_cache_fp8(key, val, code, k8, v8, slots, ks, vs)
    assert np.array_equal(kd8.cpu().numpy(), k8)
    assert np.array_equal(vd8.cpu().numpy(), v8)


def test_fp8_encode_every_f16_value_bit_exact():
    """The gfx950 converter with the explicit saturation, over all 65536 fp16
    inputs (scale 1), against the oracle's RNE/satfinite encoder."""
    allv = np.arange(65536, dtype=np.uint16)
    T, n_kv, D, BS = 512, 1, 128, 16
    key = allv.reshape(T, n_kv, D)
    slots = np.arange(T, dtype=np.int32)
    N = T // BS
    kd8 = torch.zeros(N, n_kv, D, BS, dtype=torch.uint8, device="cuda")
    vd8 = torch.zeros_like(kd8)
    tla.reshape_and_cache_fp8(dev(key, orc.F16), dev(key, orc.F16), kd8, vd8, dev(slots), 1.0, 1.0)
    torch.cuda.synchronize()
    k8 = np.zeros((N, n_kv, D, BS), np.uint8)
    v8 = np.zeros_like(k8)
    orc.reshape_and_cache_fp8(key, key, orc.F16, k8, v8, slots, 1.0, 1.0)
    got = kd8.cpu().numpy()
    t = np.arange(T)
    g = got[t // BS, 0, :, t % BS]                     # [T, D] codes per input
    w = k8[t // BS, 0, :, t % BS]
    nan = np.isnan(key.reshape(T, D).view(np.float16))
    assert np.array_equal(g[~nan], w[~nan])
    assert ((g[nan] & 0x7F) == 0x7F).all()            # NaN in, an E4M3 NaN out


@pytest.mark.parametrize("code", [orc.F16, orc.BF16, orc.F32])
def test_fp8_absmax_scale(code):
    rng = np.random.default_rng(4)
    x = rng.standard_normal(1_000_003).astype(np.float32) * 3
    x[123457] = -17.25
    xb = inputs.encode(x, code)
    out = torch.zeros(1, dtype=torch.float32, device="cuda")
    tla.fp8_absmax_scale(dev(xb, code), out)
    torch.cuda.synchronize()
    amax = np.abs(orc.bits_to_f32(xb, code) if code != orc.F32 else xb).max()
    assert out.item() == np.float32(amax) / np.float32(448.0)
    zero = torch.zeros(1000, dtype=torch.float16, device="cuda")
    tla.fp8_absmax_scale(zero, out)
    torch.cuda.synchronize()
    assert out.item() == 0.0


@pytest.mark.parametrize("scale", [1.0, 0.5, 1.0 / 448.0, 3.7])
def test_convert_fp8_every_f16_value(scale):
    """convert_fp8 (cache_kernels.cu:286-295) over all 65 536 fp16 bit
    patterns: e4m3(float(x) * scale) with RNE and saturation, NaN kept, as
    the oracle's encoder (pinned against torch and by brute force)."""
    bits = np.arange(65536, dtype=np.uint16)
    want = np.empty(65536, np.uint8)
    orc.lib.orc_convert(orc.ptr(bits), orc.F16, orc.ptr(want), orc.FP8, bits.size, scale)
    x = dev(bits, orc.F16)
    out = torch.full((65536,), 0xAB, dtype=torch.uint8, device="cuda")
    print(f"case convert_fp8 f16 scale={scale}", flush=True)
    tla.convert_fp8(out, x, scale)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    nan = (want & 0x7F) == 0x7F
    assert np.array_equal(got[~nan], want[~nan])
    assert ((got[nan] & 0x7F) == 0x7F).all()


@pytest.mark.parametrize("code", [orc.BF16, orc.F32])
def test_convert_fp8_other_sources_and_unaligned_tails(code):
    """bf16 / f32 sources; a 16-byte-aligned call and calls at odd offsets
    and lengths (the element-by-element path), bytes past n untouched."""
    rng = np.random.default_rng(66)
    x = (rng.standard_normal(10000) * np.float32(100.0)).astype(np.float32)
    x[:6] = [np.inf, -np.inf, np.nan, 1e-9, -449.0, 600.0]
    xb = inputs.encode(x, code)
    xf = orc.bits_to_f32(xb, code) if code != orc.F32 else xb
    want = orc.f32_to_e4m3(xf, np.float32(0.25))
    xd = dev(xb, code)
    for off, n in ((0, 10000), (1, 9997), (3, 33), (8, 17)):
        out = torch.full((10016,), 0xAB, dtype=torch.uint8, device="cuda")
        print(f"case convert_fp8 code={code} off={off} n={n}", flush=True)
        tla.convert_fp8(out[off:], xd[off:], 0.25, n=n)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        w = want[off:off + n]
        g = got[off:off + n]
        nan = (w & 0x7F) == 0x7F
        assert np.array_equal(g[~nan], w[~nan]) and ((g[nan] & 0x7F) == 0x7F).all()
        assert (got[:off] == 0xAB).all() and (got[off + n:] == 0xAB).all()
