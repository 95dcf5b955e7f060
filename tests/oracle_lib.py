"""ctypes binding of the CPU oracle (oracle/libtloracle.so).

Test infrastructure: the checker that tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg compare the HIP library against.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(ROOT, "oracle", "libtloracle.so")

F32, F16, BF16, FP8 = 0, 1, 2, 32
MODULO, GROUPED = 0, 1
KIVI_PAGE_BYTES = 5120
KIVI_PAGE_BYTES_INT8 = 9216


def kivi_page_bytes(bits: int) -> int:
    return KIVI_PAGE_BYTES_INT8 if bits == 8 else KIVI_PAGE_BYTES
KIVI_PAGE_TOKENS = 32

if not os.path.exists(LIB_PATH):
    raise RuntimeError(f"{LIB_PATH} missing: build it with `make -C oracle`")
_lib = ctypes.CDLL(LIB_PATH)

_P, _I, _F, _D = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_double
_lib.orc_f32_to_f16.restype = ctypes.c_uint16
_lib.orc_f32_to_f16.argtypes = [_F]
_lib.orc_f16_to_f32.restype = _F
_lib.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
_lib.orc_f32_to_bf16.restype = ctypes.c_uint16
_lib.orc_f32_to_bf16.argtypes = [_F]
_lib.orc_f32_to_e4m3.restype = ctypes.c_uint8
_lib.orc_f32_to_e4m3.argtypes = [_F]
_lib.orc_e4m3_to_f32.restype = _F
_lib.orc_e4m3_to_f32.argtypes = [ctypes.c_uint8]
_lib.orc_convert.argtypes = [_P, _I, _P, _I, ctypes.c_int64, _F]
_lib.orc_reshape_and_cache.argtypes = [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I]
_lib.orc_reshape_and_cache_fp8.argtypes = [_P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _F, _F]
_lib.orc_rope_reshape_and_cache.argtypes = [_P] * 10 + [_I] * 9
_lib.orc_rms_norm.argtypes = [_P, _P, _P, _P, _I, _I, _F, _I]
_lib.orc_layer_norm.argtypes = [_P, _P, _P, _P, _I, _I, _F, _I]
_lib.orc_act_and_mul.argtypes = [_P, _P, _P, ctypes.c_int64, _I, _I]
_lib.orc_vq_encode.argtypes = [_P, _P, _P, ctypes.c_int64, _I, _I]
_lib.orc_vq_decode.argtypes = [_P, _P, _P, ctypes.c_int64, _I, _I]
_lib.orc_vq_kmeans.argtypes = [_P, _P, ctypes.c_int64, _I, _I, _I]
_lib.orc_copy_blocks.argtypes = [_P, _P, _P, _I, _I, ctypes.c_int64]
_lib.orc_swap_blocks.argtypes = [_P, _P, _P, _I, _I, _I, ctypes.c_int64, _I]
_lib.orc_paged_attention.argtypes = [_P, _P, _I, _P, _P, _I, _F, _F, _P, _I, _P, _I, _I, _I, _I, _I, _F, _I, _I]
_lib.orc_paged_attention_f32.argtypes = [_P, _I, _P, _I, _P, _P, _I, _F, _F, _P, _I, _P, _I, _I, _I, _I, _I, _F, _I, _I]
_lib.orc_kivi_paged_attention_f32.argtypes = [_P, _P, _P, _P, _I, _I, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _F,
                                              _I, _I, _I]
_lib.orc_paged_attention_literal_v1.argtypes = [_P, _P, _P, _P, _I, _P, _I, _P, _I, _I, _I, _I, _I, _F]
_lib.orc_chunked_prefill.argtypes = [_P, _P, _I, _P, _P, _P, _I, _P, _I, _P, _I, _I, _I, _I, _I, _F, _I]
_lib.orc_kivi_compressed_bytes.restype = ctypes.c_size_t
_lib.orc_kivi_compressed_bytes.argtypes = [_I, _I, _I]
_lib.orc_kivi_params_supported.restype = _I
_lib.orc_kivi_params_supported.argtypes = [_I, _I, _I]
_lib.orc_kivi_compress.argtypes = [_P, _P, _I, _I, _I, _I]
_lib.orc_kivi_decompress.argtypes = [_P, _P, _I, _I, _I, _I]
_lib.orc_kivi_quant_group.argtypes = [_P, _I, _P, _P, _P]
_lib.orc_kivi_page_quantize.argtypes = [_P, _P, _P]
_lib.orc_kivi_page_dequant.argtypes = [_P, _P, _P]
_lib.orc_kivi_quantized_len.restype = _I
_lib.orc_kivi_quantized_len.argtypes = [_I, _I]
_lib.orc_kivi_build_pages.argtypes = [_P, _P, _P, _I, _P, _I, _I, _I, _I, _P, _P, _I, _I]
_lib.orc_kivi_paged_attention.argtypes = [_P, _P, _I, _P, _P, _I, _I, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _F, _I]
_lib.orc_kivi_page_bytes.restype = ctypes.c_size_t
_lib.orc_kivi_page_bytes.argtypes = [_I]
_lib.orc_kivi_quant_group_levels.argtypes = [_P, _I, _I, _P, _P, _P]
_lib.orc_kivi_page_quantize_bits.argtypes = [_P, _P, _P, _I]
_lib.orc_kivi_page_dequant_bits.argtypes = [_P, _P, _P, _I]
_lib.orc_kivi_build_pages_bits.argtypes = [_P, _P, _P, _I, _P, _I, _I, _I, _I, _P, _P, _I, _I, _I]
_lib.orc_kivi_paged_attention_bits.argtypes = [_P, _P, _I, _P, _P, _I, _I, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I,
                                               _F, _I, _I]
_lib.orc_kivi_paged_attention_pre_rope.argtypes = [_P, _P, _I, _P, _P, _I, _I, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I,
                                                  _F, _I, _I, _P, _P, _I, _I]

lib = _lib


def ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle needs contiguous arrays"
    return a.ctypes.data_as(ctypes.c_void_p)


def dtype_of(a: np.ndarray, hint: int | None = None) -> int:
    if hint is not None:
        return hint
    if a.dtype == np.float32:
        return F32
    if a.dtype == np.float16:
        return F16
    raise ValueError("pass the dtype code for bit-pattern arrays")


# ---- scalar / array conversions ------------------------------------------

def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    _lib.orc_convert(ptr(x), F32, ptr(out), F16, x.size, 1.0)
    return out


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    _lib.orc_convert(ptr(x), F32, ptr(out), BF16, x.size, 1.0)
    return out


def bits_to_f32(bits: np.ndarray, code: int, mul: float = 1.0) -> np.ndarray:
    bits = np.ascontiguousarray(bits)
    out = np.empty(bits.shape, np.float32)
    _lib.orc_convert(ptr(bits), code, ptr(out), F32, bits.size, mul)
    return out


def f32_to_e4m3(x: np.ndarray, mul: float = 1.0) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint8)
    _lib.orc_convert(ptr(x), F32, ptr(out), FP8, x.size, mul)
    return out


# ---- hot-path restatements -----------------------------------------------

def reshape_and_cache(key, value, k_cache, v_cache, slots):
    T, n_kv, D = key.shape
    _lib.orc_reshape_and_cache(ptr(key), ptr(value), ptr(k_cache), ptr(v_cache), ptr(slots), T,
                               n_kv, D, k_cache.shape[3], key.dtype.itemsize)


def rope_reshape_and_cache(q, q_out, key, value, k_cache, v_cache, slots, positions, cos_t, sin_t, code,
                           style):
    """In place on q_out and the pools (numpy, dtype code F16 / BF16 as uint16, F32)."""
    T, n_kv, D = key.shape
    H = 0 if q is None else q.shape[1]
    _lib.orc_rope_reshape_and_cache(None if q is None else ptr(q), None if q_out is None else ptr(q_out),
                                    ptr(key), ptr(value), ptr(k_cache), ptr(v_cache), ptr(slots),
                                    ptr(positions), ptr(cos_t), ptr(sin_t), cos_t.shape[0], T, H, n_kv, D,
                                    k_cache.shape[3], k_cache.shape[0], code, style)


def rms_norm(x, w, eps, code, residual=None):
    """Returns out (same storage as x); residual (if given) is updated in place."""
    out = np.zeros_like(x)
    _lib.orc_rms_norm(ptr(out), None if residual is None else ptr(residual), ptr(x), ptr(w), x.shape[0],
                      x.shape[1], eps, code)
    return out


def layer_norm(x, w, b, eps, code):
    out = np.zeros_like(x)
    _lib.orc_layer_norm(ptr(out), ptr(x), ptr(w), ptr(b), x.shape[0], x.shape[1], eps, code)
    return out


def act_and_mul(gate, up, act, code):
    out = np.zeros_like(gate)
    _lib.orc_act_and_mul(ptr(out), ptr(gate), ptr(up), gate.size, act, code)
    return out


def vq_encode(kv_bits, book_bits):
    """fp16 bits kv [..., D], book [K, D] -> uint16 indices [n]."""
    D = book_bits.shape[1]
    kv = np.ascontiguousarray(kv_bits, np.uint16)
    idx = np.zeros(kv.size // D, np.uint16)
    _lib.orc_vq_encode(ptr(kv), ptr(np.ascontiguousarray(book_bits, np.uint16)), ptr(idx), idx.size, D,
                       book_bits.shape[0])
    return idx


def vq_decode(out_bits, book_bits, idx):
    D = book_bits.shape[1]
    _lib.orc_vq_decode(ptr(out_bits), ptr(np.ascontiguousarray(book_bits, np.uint16)),
                       ptr(np.ascontiguousarray(idx, np.uint16)), idx.size, D, book_bits.shape[0])


def vq_kmeans(data_bits, book_bits, iterations):
    """In place on book_bits (uint16 [K, D])."""
    D = book_bits.shape[1]
    data = np.ascontiguousarray(data_bits, np.uint16)
    _lib.orc_vq_kmeans(ptr(data), ptr(book_bits), data.size // D, book_bits.shape[0], D, iterations)


def copy_blocks(k_cache, v_cache, mapping):
    """In place on numpy pools [N, ...]; mapping int32 [P, 2]."""
    nb = k_cache.shape[0]
    _lib.orc_copy_blocks(ptr(k_cache), ptr(v_cache), ptr(mapping), mapping.shape[0], nb,
                         k_cache[0].nbytes)


def swap_blocks(cache, host_cache, mapping, direction):
    _lib.orc_swap_blocks(ptr(cache), ptr(host_cache), ptr(mapping), mapping.shape[0], cache.shape[0],
                         host_cache.shape[0], cache[0].nbytes, direction)


def reshape_and_cache_fp8(key, value, src_code, k_cache, v_cache, slots, k_scale, v_scale):
    T, n_kv, D = key.shape
    _lib.orc_reshape_and_cache_fp8(ptr(key), ptr(value), src_code, ptr(k_cache), ptr(v_cache),
                                   ptr(slots), T, n_kv, D, k_cache.shape[3], k_scale, v_scale)


def paged_attention(q, q_code, k_cache, v_cache, kv_code, tables, seq_lens, num_kv_heads, scale,
                    gqa_map=GROUPED, partition_tokens=0, k_scale=1.0, v_scale=1.0):
    S, H, D = q.shape
    out = np.zeros((S, H, D), np.float64)
    _lib.orc_paged_attention(ptr(out), ptr(q), q_code, ptr(k_cache), ptr(v_cache), kv_code,
                             k_scale, v_scale, ptr(tables), tables.shape[1], ptr(seq_lens), S, H,
                             num_kv_heads, D, k_cache.shape[3], scale, gqa_map, partition_tokens)
    return out


def paged_attention_f32(q, q_code, k_cache, v_cache, kv_code, tables, seq_lens, num_kv_heads,
                        scale, gqa_map=GROUPED, threads=1, k_scale=1.0, v_scale=1.0):
    S, H, D = q.shape
    out = np.zeros((S, H, D), np.float32)
    _lib.orc_paged_attention_f32(ptr(out), F32, ptr(q), q_code, ptr(k_cache), ptr(v_cache),
                                 kv_code, k_scale, v_scale, ptr(tables), tables.shape[1],
                                 ptr(seq_lens), S, H, num_kv_heads, D, k_cache.shape[3], scale,
                                 gqa_map, threads)
    return out


def kivi_paged_attention_f32(q, pages, page_tables, k_cache, v_cache, tables, seq_lens, num_kv_heads,
                             residual_length, scale, gqa_map=GROUPED, bits=4, threads=1):
    """The CPU baseline's paged KIVI decode (fp32, threads over (seq, kv
    head)); fp16 q and output bits."""
    S, H, D = q.shape
    out = np.zeros((S, H, D), np.uint16)
    num_pages = pages.size // (num_kv_heads * kivi_page_bytes(bits))
    _lib.orc_kivi_paged_attention_f32(ptr(out), ptr(q), ptr(pages), ptr(page_tables), page_tables.shape[1],
                                      num_pages, ptr(k_cache), ptr(v_cache), ptr(tables), tables.shape[1],
                                      ptr(seq_lens), S, H, num_kv_heads, k_cache.shape[3], residual_length,
                                      scale, gqa_map, bits, threads)
    return out


def paged_attention_literal_v1(q, k_cache, v_cache, code, tables, seq_lens, num_kv_heads, scale):
    S, H, D = q.shape
    out = np.full((S, H, D), np.nan, np.float32)
    _lib.orc_paged_attention_literal_v1(ptr(out), ptr(q), ptr(k_cache), ptr(v_cache), code,
                                        ptr(tables), tables.shape[1], ptr(seq_lens), S, H,
                                        num_kv_heads, D, k_cache.shape[3], scale)
    return out


def chunked_prefill(q, q_code, cu_q_lens, k_cache, v_cache, kv_code, tables, seq_lens,
                    num_kv_heads, scale, gqa_map=GROUPED):
    T, H, D = q.shape
    out = np.zeros((T, H, D), np.float64)
    _lib.orc_chunked_prefill(ptr(out), ptr(q), q_code, ptr(cu_q_lens), ptr(k_cache),
                             ptr(v_cache), kv_code, ptr(tables), tables.shape[1], ptr(seq_lens),
                             len(seq_lens), H, num_kv_heads, D, k_cache.shape[3], scale, gqa_map)
    return out


# ---- KIVI ------------------------------------------------------------------

def kivi_compressed_bytes(head_dim, n_outliers, group_size) -> int:
    return _lib.orc_kivi_compressed_bytes(head_dim, n_outliers, group_size)


def kivi_params_supported(head_dim, n_outliers, group_size) -> bool:
    return bool(_lib.orc_kivi_params_supported(head_dim, n_outliers, group_size))


def kivi_compress(x_bits: np.ndarray, head_dim, n_outliers, group_size, out=None):
    n = x_bits.size // head_dim
    stride = kivi_compressed_bytes(head_dim, n_outliers, group_size)
    if out is None:
        out = np.zeros(max(1, n * stride), np.uint8)
    _lib.orc_kivi_compress(ptr(x_bits), ptr(out), n, head_dim, n_outliers, group_size)
    return out


def kivi_decompress(rec: np.ndarray, n_vecs, head_dim, n_outliers, group_size):
    out = np.zeros(n_vecs * head_dim, np.uint16)
    _lib.orc_kivi_decompress(ptr(rec), ptr(out), n_vecs, head_dim, n_outliers, group_size)
    return out


def kivi_quant_group(x: np.ndarray):
    x = np.ascontiguousarray(x, np.float32)
    q = np.zeros(x.size, np.uint8)
    st = np.zeros(1, np.uint16)
    ze = np.zeros(1, np.uint16)
    _lib.orc_kivi_quant_group(ptr(x), x.size, ptr(q), ptr(st), ptr(ze))
    return q, int(st[0]), int(ze[0])


def kivi_quant_group_levels(x: np.ndarray, levels: int):
    x = np.ascontiguousarray(x, np.float32)
    q = np.zeros(x.size, np.uint8)
    st = np.zeros(1, np.uint16)
    ze = np.zeros(1, np.uint16)
    _lib.orc_kivi_quant_group_levels(ptr(x), x.size, levels, ptr(q), ptr(st), ptr(ze))
    return q, int(st[0]), int(ze[0])


def kivi_page_quantize(k_tok_bits, v_tok_bits, bits=4):
    page = np.zeros(kivi_page_bytes(bits), np.uint8)
    if bits == 4:
        _lib.orc_kivi_page_quantize(ptr(k_tok_bits), ptr(v_tok_bits), ptr(page))
    else:
        _lib.orc_kivi_page_quantize_bits(ptr(k_tok_bits), ptr(v_tok_bits), ptr(page), bits)
    return page


def kivi_page_dequant(page, bits=4):
    k = np.zeros((32, 128), np.uint16)
    v = np.zeros((32, 128), np.uint16)
    if bits == 4:
        _lib.orc_kivi_page_dequant(ptr(page), ptr(k), ptr(v))
    else:
        _lib.orc_kivi_page_dequant_bits(ptr(page), ptr(k), ptr(v), bits)
    return k, v


def kivi_quantized_len(seq_len, residual_length) -> int:
    return _lib.orc_kivi_quantized_len(seq_len, residual_length)


def kivi_build_pages(k_cache, v_cache, tables, seq_lens, residual_length, pages, page_tables, bits=4):
    num_pages = pages.size // (k_cache.shape[1] * kivi_page_bytes(bits))
    if bits == 4:
        _lib.orc_kivi_build_pages(ptr(k_cache), ptr(v_cache), ptr(tables), tables.shape[1],
                                  ptr(seq_lens), len(seq_lens), k_cache.shape[1], k_cache.shape[3],
                                  residual_length, ptr(pages), ptr(page_tables), page_tables.shape[1], num_pages)
    else:
        _lib.orc_kivi_build_pages_bits(ptr(k_cache), ptr(v_cache), ptr(tables), tables.shape[1],
                                       ptr(seq_lens), len(seq_lens), k_cache.shape[1], k_cache.shape[3],
                                       residual_length, ptr(pages), ptr(page_tables), page_tables.shape[1],
                                       num_pages, bits)


def kivi_paged_attention(q, q_code, pages, page_tables, k_cache, v_cache, tables, seq_lens,
                         num_kv_heads, residual_length, scale, gqa_map=GROUPED, bits=4, pre_rope=None):
    """pre_rope = (cos_t, sin_t, style): the keys are held before RoPE and
    rotated by their positions inside attention."""
    S, H, D = q.shape
    out = np.zeros((S, H, D), np.float64)
    num_pages = pages.size // (num_kv_heads * kivi_page_bytes(bits))
    args = (ptr(out), ptr(q), q_code, ptr(pages), ptr(page_tables), page_tables.shape[1], num_pages,
            ptr(k_cache), ptr(v_cache), ptr(tables), tables.shape[1], ptr(seq_lens), S, H, num_kv_heads,
            k_cache.shape[3], residual_length, scale, gqa_map)
    if pre_rope is not None:
        cos_t, sin_t, style = pre_rope
        _lib.orc_kivi_paged_attention_pre_rope(*args, bits, ptr(cos_t), ptr(sin_t), cos_t.shape[0], style)
        return out
    if bits == 4:
        _lib.orc_kivi_paged_attention(*args)
    else:
        _lib.orc_kivi_paged_attention_bits(*args, bits)
    return out
