"""The reference-named C++ operators (include/tl_truellm_ops.h), called by
their mangled names with TrueBuffer views built here, give the same bytes as
the C ABI entry points they forward to; unsupported calls are no-ops, as in
the reference's release build."""
import ctypes
import math

import numpy as np
import pytest
import torch

import inputs
import oracle_lib as orc
import tl_attn as tla
from gpu_util import assert_close, dev

pytestmark = pytest.mark.gpu


class TrueBuffer(ctypes.Structure):
    """include/truellm/types.h:69-77."""
    _fields_ = [("data", ctypes.c_void_p), ("size_bytes", ctypes.c_size_t), ("dtype", ctypes.c_uint8),
                ("device_id", ctypes.c_int32), ("ndim", ctypes.c_int32), ("shape", ctypes.c_int64 * 4),
                ("stride", ctypes.c_int64 * 4)]


_DT = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2, torch.int32: 3, torch.uint8: 5}


def tb(t):
    """A TrueBuffer view of a contiguous CUDA tensor (strides left 0, as make_tb does)."""
    b = TrueBuffer()
    b.data = t.data_ptr()
    b.size_bytes = t.numel() * t.element_size()
    b.dtype = _DT[t.dtype]
    b.device_id = 0
    b.ndim = t.dim()
    for i in range(4):
        b.shape[i] = t.shape[i] if i < t.dim() else 1
    return b


def _fn(mangled, argtypes, restype=None):
    f = tla.lib[mangled]
    f.argtypes = argtypes
    f.restype = restype
    return f


_R = ctypes.POINTER(TrueBuffer)
_S = ctypes.c_void_p
V1 = _fn("_Z18paged_attention_v1RN7truellm10TrueBufferERKS0_S3_S3_S3_S3_ifiiP12ihipStream_t",
         [_R] * 6 + [ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_int, _S])
V2 = _fn("_Z18paged_attention_v2RN7truellm10TrueBufferES1_S1_S1_RKS0_S3_S3_S3_S3_ifiiiP12ihipStream_t",
         [_R] * 9 + [ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_int, _S])
RC = _fn("_Z17reshape_and_cacheRKN7truellm10TrueBufferES2_RS0_S2_P12ihipStream_t", [_R] * 4 + [_S])
CB = _fn("_Z11copy_blocksRN7truellm10TrueBufferERKS0_P12ihipStream_t", [_R] * 2 + [_S])
SB = _fn("_Z11swap_blocksRN7truellm10TrueBufferES1_RKS0_iP12ihipStream_t", [_R] * 3 + [ctypes.c_int, _S])
KC = _fn("_ZN7truellm13kivi_compressEPK6__halfPhiiiiP12ihipStream_t",
         [_S, _S] + [ctypes.c_int] * 4 + [_S])
KD = _fn("_ZN7truellm15kivi_decompressEPKhP6__halfiiiiP12ihipStream_t",
         [_S, _S] + [ctypes.c_int] * 4 + [_S])


def _stream():
    return torch.cuda.current_stream().cuda_stream


def test_v1_v2_shims_equal_c_abi():
    case = inputs.make_paged_case(inputs.SEEDS[0], 4, 32, 8, 128, 16, [1000, 17, 513, 2048], orc.F16)
    q, k, v = dev(case.q, orc.F16), dev(case.k_cache, orc.F16), dev(case.v_cache, orc.F16)
    bt, sl = dev(case.tables), dev(case.seq_lens)
    a = torch.full_like(q, float("nan"))
    b = torch.full_like(q, float("nan"))
    print("case shim v1", flush=True)
    V1(tb(a), tb(q), tb(k), tb(v), tb(bt), tb(sl), 8, case.scale, 128, 16, _stream())
    tla.paged_attention_v1(b, q, k, v, bt, sl, 8, case.scale, 128, 16)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    P = tla.v2_num_partitions(2048, 16)
    es = torch.zeros(4, 32, P, device="cuda")
    ml = torch.zeros(4, 32, P, device="cuda")
    tmp = torch.zeros(4, 32, P, 128, dtype=torch.float16, device="cuda")
    c = torch.full_like(q, float("nan"))
    print("case shim v2", flush=True)
    V2(tb(c), tb(es), tb(ml), tb(tmp), tb(q), tb(k), tb(v), tb(bt), tb(sl), 8, case.scale, 128, 16, 2048,
       _stream())
    torch.cuda.synchronize()
    assert (c.float() - b.float()).abs().max().item() < 4e-3


def test_v1_shim_unsupported_is_a_no_op():
    """Head size 72 is in no dispatch table (the reference asserts,
    paged_attention_v1.cu:212): the operator leaves out untouched."""
    case = inputs.make_paged_case(inputs.SEEDS[0], 2, 8, 2, 72, 16, [100, 50], orc.F16)
    q, k, v = dev(case.q, orc.F16), dev(case.k_cache, orc.F16), dev(case.v_cache, orc.F16)
    bt, sl = dev(case.tables), dev(case.seq_lens)     # held: a view of a freed tensor may alias the next
    out = torch.full_like(q, 7.0)
    V1(tb(out), tb(q), tb(k), tb(v), tb(bt), tb(sl), 2, case.scale, 72, 16, _stream())
    torch.cuda.synchronize()
    assert (out == 7.0).all()
    assert "head_size=72" in tla.last_error()


@pytest.mark.parametrize("D", [80, 96])
def test_v1_shim_heads_80_and_96(D):
    """The reference's F16 heads 80 and 96 (paged_attention_v1.cu:200-201)
    through the C++ operator, against the oracle (MODULO map, as the
    reference indexes)."""
    case = inputs.make_paged_case(inputs.SEEDS[0] + D, 3, 8, 2, D, 16, [100, 50, 700], orc.F16)
    q, k, v = dev(case.q, orc.F16), dev(case.k_cache, orc.F16), dev(case.v_cache, orc.F16)
    bt, sl = dev(case.tables), dev(case.seq_lens)
    out = torch.full_like(q, float("nan"))
    print(f"case v1 shim D={D}", flush=True)
    V1(tb(out), tb(q), tb(k), tb(v), tb(bt), tb(sl), 2, case.scale, D, 16, _stream())
    torch.cuda.synchronize()
    ref = orc.paged_attention(case.q, orc.F16, case.k_cache, case.v_cache, orc.F16, case.tables, case.seq_lens,
                              2, case.scale, orc.MODULO)
    assert_close(out, ref, orc.F16, 2e-3, f"v1 shim D={D}")


def test_reshape_and_cache_shim_equals_c_abi():
    rng = np.random.default_rng(3)
    T, n_kv, D, BS, N = 37, 8, 128, 16, 40
    key = torch.from_numpy(rng.standard_normal((T, n_kv, D), dtype=np.float32)).to(torch.bfloat16).cuda()
    val = torch.from_numpy(rng.standard_normal((T, n_kv, D), dtype=np.float32)).to(torch.bfloat16).cuda()
    slots = torch.from_numpy(rng.permutation(N * BS)[:T].astype(np.int32)).cuda()
    slots[5] = -1
    kv_a = torch.zeros(2 * N, n_kv, D, BS, dtype=torch.bfloat16, device="cuda")
    kv_b = torch.zeros_like(kv_a)
    print("case shim reshape", flush=True)
    RC(tb(key), tb(val), tb(kv_a), tb(slots), _stream())
    tla.reshape_and_cache(key, val, kv_b, slots)
    torch.cuda.synchronize()
    assert torch.equal(kv_a.view(torch.int16), kv_b.view(torch.int16))
    assert kv_a.view(torch.int16).abs().sum().item() > 0


def test_kivi_codec_shims_equal_c_abi_and_no_op_when_unsupported():
    rng = np.random.default_rng(4)
    n, D, O, G = 300, 128, 8, 16
    x = torch.from_numpy(rng.standard_normal((n, D), dtype=np.float32)).half().cuda()
    stride = tla.kivi_compressed_bytes(D, O, G)
    a = torch.zeros(n, stride, dtype=torch.uint8, device="cuda")
    b = torch.zeros_like(a)
    print("case shim kivi", flush=True)
    KC(x.data_ptr(), a.data_ptr(), n, D, O, G, _stream())
    tla.kivi_compress(x, b, n, D, O, G)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    ya = torch.zeros_like(x)
    yb = torch.zeros_like(x)
    KD(a.data_ptr(), ya.data_ptr(), n, D, O, G, _stream())
    tla.kivi_decompress(b, yb, n, D, O, G)
    torch.cuda.synchronize()
    assert torch.equal(ya.view(torch.int16), yb.view(torch.int16))
    untouched = torch.full_like(a, 0xAB)
    KC(x.data_ptr(), untouched.data_ptr(), n, 200, O, G, _stream())      # head_dim > 128: no-op
    torch.cuda.synchronize()
    assert (untouched == 0xAB).all()


def test_manifest_initialize_accepts_this_device():
    class M(ctypes.Structure):
        _fields_ = [("abi_version", ctypes.c_uint32), ("name", ctypes.c_char_p), ("version", ctypes.c_char_p),
                    ("category", ctypes.c_int), ("min_sm_major", ctypes.c_uint32),
                    ("min_sm_minor", ctypes.c_uint32),
                    ("initialize", ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p)),
                    ("shutdown", ctypes.CFUNCTYPE(None, ctypes.c_void_p)), ("kernel_state", ctypes.c_void_p)]
    fn = tla.lib.truellm_kernel_init
    fn.restype = ctypes.POINTER(M)
    m = fn().contents
    torch.cuda.synchronize()
    assert m.initialize(None) == 0
    m.shutdown(None)


def test_block_shims_equal_c_abi():
    """copy_blocks on the [2N, n_kv, d, bs] buffer (K blocks then V) and
    swap_blocks to a pinned host buffer, by their reference names."""
    g = torch.Generator(device="cuda").manual_seed(5)
    N, n_kv, D, BS = 48, 8, 128, 16
    kv_a = torch.randn(2 * N, n_kv, D, BS, generator=g, device="cuda", dtype=torch.float16)
    kv_b = kv_a.clone()
    m = torch.tensor([[3, 40], [7, 1], [12, 13], [47, 0]], dtype=torch.int32, device="cuda")
    print("case shim copy_blocks", flush=True)
    CB(tb(kv_a), tb(m), _stream())
    tla.copy_blocks(kv_b[:N], kv_b[N:], m)
    torch.cuda.synchronize()
    assert torch.equal(kv_a.view(torch.int16), kv_b.view(torch.int16))
    assert torch.equal(kv_a[40], kv_a[3]) and torch.equal(kv_a[N + 40], kv_a[N + 3])
    host = torch.zeros(6, n_kv, D, BS, dtype=torch.float16, pin_memory=True)
    sm = torch.tensor([[5, 2], [90, 4]], dtype=torch.int32, device="cuda")
    print("case shim swap_blocks", flush=True)
    SB(tb(kv_a), tb(host), tb(sm), 0, _stream())
    torch.cuda.synchronize()
    assert torch.equal(host[2], kv_a[5].cpu()) and torch.equal(host[4], kv_a[90].cpu())


CF8 = _fn("_Z11convert_fp8RN7truellm10TrueBufferERKS0_fP12ihipStream_t", [_R, _R, ctypes.c_float, _S])


def test_convert_fp8_shim_equals_c_abi():
    """The reference-named convert_fp8 over a [blocks, n_kv, d, bs] fp16
    view (every element of the view's shape) gives the C ABI's bytes."""
    x = (torch.randn(9, 4, 128, 16, device="cuda") * 50).to(torch.float16)
    a = torch.zeros(x.numel(), dtype=torch.uint8, device="cuda")
    b = torch.zeros_like(a)
    print("case convert_fp8 shim", flush=True)
    CF8(tb(a.view(9, 4, 128, 16)), tb(x), 1.0 / 3.0, _stream())
    tla.convert_fp8(b, x, 1.0 / 3.0)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and (a != 0).any()
