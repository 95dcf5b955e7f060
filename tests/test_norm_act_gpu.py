"""RMSNorm / fused add + RMSNorm / LayerNorm and the gated activations on
the GPU against the oracle (within one output ulp), the reference tests'
cases, and the reference-named operators."""
import ctypes

import numpy as np
import pytest
import torch

import inputs
import oracle_lib as orc
import tl_attn as tla
from gpu_util import dev, host_bits, host_f64

pytestmark = pytest.mark.gpu

ULP = {orc.F16: 2.0 ** -10, orc.BF16: 2.0 ** -7, orc.F32: 2.0 ** -22}


def _close(got_t, ref_bits, code, ulps=1.0):
    ref = orc.bits_to_f32(ref_bits, code).astype(np.float64) if code != orc.F32 else ref_bits.astype(np.float64)
    got = host_f64(got_t)
    tol = ulps * ULP[code] * np.maximum(np.abs(ref), 2.0 ** -14) + 1e-6
    bad = np.abs(got - ref) > tol
    assert not bad.any(), (np.argwhere(bad)[:5], got[bad][:5], ref[bad][:5])


SHAPES = [(64, 4096), (3, 96), (1, 8), (17, 5000)]


@pytest.mark.parametrize("code", [orc.F16, orc.BF16, orc.F32])
@pytest.mark.parametrize("T,H", SHAPES)
def test_rms_norm_and_fused_add(code, T, H):
    rng = np.random.default_rng(T * 31 + H)
    x = inputs.encode(rng.standard_normal((T, H), dtype=np.float32) * 3, code)
    res = inputs.encode(rng.standard_normal((T, H), dtype=np.float32), code)
    w = inputs.encode(1 + 0.2 * rng.standard_normal(H, dtype=np.float32), code)
    xd, wd = dev(x, code), dev(w, code)
    out = torch.zeros_like(xd)
    print(f"case rms_norm code={code} T={T} H={H}", flush=True)
    tla.rms_norm(out, xd, wd, 1e-6)
    torch.cuda.synchronize()
    _close(out, orc.rms_norm(x, w, 1e-6, code), code)
    rd = dev(res, code)
    out2 = torch.zeros_like(xd)
    tla.fused_add_rms_norm(out2, rd, xd, wd, 1e-6)
    torch.cuda.synchronize()
    r_ref = res.copy()
    ref2 = orc.rms_norm(x, w, 1e-6, code, residual=r_ref)
    assert np.array_equal(host_bits(rd), r_ref)              # the residual update is exact
    _close(out2, ref2, code)


@pytest.mark.parametrize("code", [orc.F16, orc.BF16, orc.F32])
@pytest.mark.parametrize("T,H", SHAPES)
def test_layer_norm(code, T, H):
    rng = np.random.default_rng(T * 37 + H)
    x = inputs.encode(rng.standard_normal((T, H), dtype=np.float32) + 0.5, code)
    w = inputs.encode(rng.standard_normal(H, dtype=np.float32), code)
    b = inputs.encode(rng.standard_normal(H, dtype=np.float32), code)
    out = torch.zeros_like(dev(x, code))
    print(f"case layer_norm code={code} T={T} H={H}", flush=True)
    tla.layer_norm(out, dev(x, code), dev(w, code), dev(b, code), 1e-5)
    torch.cuda.synchronize()
    ref = orc.layer_norm(x, w, b, 1e-5, code)
    # near-zero outputs (w * norm + b cancelling) are bounded by the inputs' scale
    _close(out, ref, code, ulps=2.0)


@pytest.mark.parametrize("act", [tla.ACT_SILU, tla.ACT_GELU, tla.ACT_GELU_TANH])
@pytest.mark.parametrize("code", [orc.F16, orc.BF16, orc.F32])
def test_act_and_mul(act, code):
    rng = np.random.default_rng(80 + act)
    n = 4 * 14336 + 7
    g = inputs.encode(rng.standard_normal(n, dtype=np.float32) * 4, code)
    u = inputs.encode(rng.standard_normal(n, dtype=np.float32), code)
    out = torch.zeros_like(dev(g, code))
    print(f"case act={act} code={code}", flush=True)
    tla.act_and_mul(out, dev(g, code), dev(u, code), act)
    torch.cuda.synchronize()
    # the activation is rounded to the dtype before the product: a one-ulp
    # difference in exp / erf / tanh can move that rounding by one ulp
    _close(out, orc.act_and_mul(g, u, act, code), code, ulps=2.5)


def test_norm_act_reference_known_answers_on_gpu():
    """test_vllm_kernels.cpp:128-253 through the library."""
    T, H = 2, 8
    x = torch.tensor(0.1 * (np.arange(T * H) + 1), dtype=torch.float32, device="cuda").view(T, H)
    w = torch.tensor(1.0 - 0.05 * np.arange(H), dtype=torch.float32, device="cuda")
    out = torch.zeros_like(x)
    tla.rms_norm(out, x, w, 1e-5)
    xd = x.double().cpu()
    want = xd / torch.sqrt((xd ** 2).mean(1, keepdim=True) + 1e-5) * w.double().cpu()
    torch.cuda.synchronize()
    assert torch.allclose(out.double().cpu(), want, atol=1e-4, rtol=0)
    u = torch.full((1, 32), 2.5, device="cuda")
    o = torch.zeros_like(u)
    tla.rms_norm(o, u, torch.ones(32, device="cuda"), 0.0)
    g = torch.tensor(-1.0 + 0.07 * np.arange(64), dtype=torch.float32, device="cuda").view(4, 16)
    up = torch.tensor(0.25 + 0.03 * np.arange(64), dtype=torch.float32, device="cuda").view(4, 16)
    s = torch.zeros_like(g)
    tla.act_and_mul(s, g, up)
    z = torch.zeros(2, 64, device="cuda")
    tla.act_and_mul(z, torch.arange(-64, 64, dtype=torch.float32, device="cuda").view(2, 64), torch.zeros(2, 64,
                    device="cuda"))
    torch.cuda.synchronize()
    assert torch.allclose(o, torch.ones_like(o), atol=1e-4)
    gd = g.double().cpu()
    assert torch.allclose(s.double().cpu(), gd / (1 + torch.exp(-gd)) * up.double().cpu(), atol=1e-5, rtol=0)
    assert not z.any()


class _TB(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("size_bytes", ctypes.c_size_t), ("dtype", ctypes.c_uint8),
                ("device_id", ctypes.c_int32), ("ndim", ctypes.c_int32), ("shape", ctypes.c_int64 * 4),
                ("stride", ctypes.c_int64 * 4)]


def _tb(t):
    b = _TB()
    b.data = t.data_ptr()
    b.size_bytes = t.numel() * t.element_size()
    b.dtype = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[t.dtype]
    b.ndim = t.dim()
    for i in range(4):
        b.shape[i] = t.shape[i] if i < t.dim() else 1
    return b


def test_norm_act_shims_equal_c_abi():
    R = ctypes.POINTER(_TB)
    rms = tla.lib["_Z8rms_normRN7truellm10TrueBufferERKS0_S3_fP12ihipStream_t"]
    rms.argtypes, rms.restype = [R, R, R, ctypes.c_float, ctypes.c_void_p], None
    silu = tla.lib["_Z12silu_and_mulRN7truellm10TrueBufferERKS0_S3_P12ihipStream_t"]
    silu.argtypes, silu.restype = [R, R, R, ctypes.c_void_p], None
    g = torch.Generator(device="cuda").manual_seed(9)
    x = torch.randn(8, 4096, generator=g, device="cuda", dtype=torch.bfloat16)
    w = torch.randn(4096, generator=g, device="cuda", dtype=torch.bfloat16)
    a, b = torch.zeros_like(x), torch.zeros_like(x)
    st = torch.cuda.current_stream().cuda_stream
    print("case norm shims", flush=True)
    rms(_tb(a), _tb(x), _tb(w), 1e-5, st)
    tla.rms_norm(b, x, w, 1e-5)
    u = torch.randn_like(x)
    c, d = torch.zeros_like(x), torch.zeros_like(x)
    silu(_tb(c), _tb(x), _tb(u), st)
    tla.act_and_mul(d, x, u, tla.ACT_SILU)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert torch.equal(c.view(torch.int16), d.view(torch.int16))
