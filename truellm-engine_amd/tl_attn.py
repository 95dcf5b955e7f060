"""Python host mirror of truellm-engine's attention operator interface over
the gfx950 C ABI (include/tl_attn.h, libtlattn.so).

The reference exposes free C++ functions taking TrueBuffer views
(paged_attention_v1.cu:177, paged_attention_v2.cu:176, cache_kernels.cu:202,
kivi_cache.cu:205-239).  The functions here take torch tensors on the GPU in
the same roles and with the same argument meaning; shapes are read from the
tensors the way the reference reads TrueBuffer.shape.  They launch on the
current torch stream and raise TLError when the library reports an error.

torch is only the device-memory and stream plumbing: every computation runs
in the HIP kernels of libtlattn.so.  There is no fallback: importing this
module without the built library raises.
"""
from __future__ import annotations

import ctypes
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libtlattn.so")
HEADER_DIR = os.path.join(os.path.dirname(_HERE), "include")

# tl_dtype (mirrors truellm::DataType for the first three)
F32, F16, BF16, FP8_E4M3 = 0, 1, 2, 32
# tl_gqa_map
GQA_MODULO, GQA_GROUPED = 0, 1
# tl_status
OK, ERR_INVALID_ARGUMENT, ERR_NOT_IMPLEMENTED, ERR_BACKEND, ERR_INTERNAL = 0, 1, 3, 5, 99

KIVI_MAX_HEAD_DIM = 128
KIVI_MAX_OUTLIERS = 64


class TLError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"tl_status {code}: {msg}")
        self.code = code


class DecodeDesc(ctypes.Structure):
    _fields_ = [
        ("num_seqs", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_size", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("max_blocks_per_seq", ctypes.c_int32),
        ("num_blocks", ctypes.c_int32),
        ("q_dtype", ctypes.c_int32),
        ("kv_dtype", ctypes.c_int32),
        ("gqa_map", ctypes.c_int32),
        ("partition_tokens", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("k_scale", ctypes.c_float),
        ("v_scale", ctypes.c_float),
    ]


class KiviDesc(ctypes.Structure):
    _fields_ = [
        ("num_seqs", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_size", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("max_blocks_per_seq", ctypes.c_int32),
        ("num_blocks", ctypes.c_int32),
        ("max_pages_per_seq", ctypes.c_int32),
        ("num_pages", ctypes.c_int32),
        ("residual_length", ctypes.c_int32),
        ("gqa_map", ctypes.c_int32),
        ("partition_pages", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("bits", ctypes.c_int32),
        ("pre_rope_keys", ctypes.c_int32),
        ("build_ahead", ctypes.c_int32),
    ]


KIVI_PAGE_TOKENS = 32
KIVI_PAGE_BYTES = 5120
KIVI_PAGE_BYTES_INT8 = 9216


def kivi_page_bytes(bits: int = 4) -> int:
    """Page bytes per kv head of a KIVI page pool (tl_kivi_page_bytes)."""
    return int(lib.tl_kivi_page_bytes(bits))


class PrefillDesc(ctypes.Structure):
    _fields_ = [
        ("num_seqs", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_size", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("max_blocks_per_seq", ctypes.c_int32),
        ("num_blocks", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("gqa_map", ctypes.c_int32),
        ("num_prefill_seqs", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("kv_dtype", ctypes.c_int32),
        ("k_scale", ctypes.c_float),
        ("v_scale", ctypes.c_float),
    ]

_P = ctypes.c_void_p
_I = ctypes.c_int32
_F = ctypes.c_float
_SIG = {
    "tl_abi_version": (ctypes.c_int, []),
    "tl_last_error_string": (ctypes.c_char_p, []),
    "tl_paged_attention_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(DecodeDesc), _I]),
    "tl_paged_attention_decode": (ctypes.c_int, [ctypes.POINTER(DecodeDesc), _P, _P, _P, _P, _P, _P, _I, _P, ctypes.c_size_t, _P]),
    "tl_paged_attention_decode_noalloc": (ctypes.c_int, [ctypes.POINTER(DecodeDesc), _P, _P, _P, _P, _P, _P, _I, _P]),
    "tl_paged_attention_v1": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _I, _I, _P]),
    "tl_paged_attention_v2": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _I, _I, _I, _P]),
    "tl_paged_attention_v2_capacity": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _I,
                                                      _I, _I, _I, _P]),
    "tl_paged_attention_v2_partitions": (_I, [_I, _I, _I, _I, _I, _I, _I, _P]),
    "tl_paged_attention_v2_capacity_partitions": (_I, [_I, _I, _I, _I, _I, _I, _I, _I, _P]),
    "tl_reshape_and_cache": (ctypes.c_int, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "tl_reshape_and_cache_fp8": (ctypes.c_int, [_P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _F, _F, _P]),
    "tl_rope_reshape_and_cache": (ctypes.c_int, [_P] * 10 + [_I] * 9 + [_P]),
    "tl_rms_norm": (ctypes.c_int, [_P, _P, _P, _I, _I, _F, _I, _P]),
    "tl_fused_add_rms_norm": (ctypes.c_int, [_P, _P, _P, _P, _I, _I, _F, _I, _P]),
    "tl_layer_norm": (ctypes.c_int, [_P, _P, _P, _P, _I, _I, _F, _I, _P]),
    "tl_act_and_mul": (ctypes.c_int, [_P, _P, _P, ctypes.c_int64, _I, _I, _P]),
    "tl_vq_encode": (ctypes.c_int, [_P, _P, _P, _I, _I, _I, _P]),
    "tl_vq_decode": (ctypes.c_int, [_P, _P, _P, _I, _I, _I, _P]),
    "tl_vq_kmeans_workspace_bytes": (ctypes.c_size_t, [_I, _I, _I]),
    "tl_vq_kmeans": (ctypes.c_int, [_P, _P, _I, _I, _I, _I, _P, ctypes.c_size_t, _P]),
    "tl_copy_blocks": (ctypes.c_int, [_P, _P, _P, _I, _I, ctypes.c_int64, _P]),
    "tl_swap_blocks": (ctypes.c_int, [_P, _P, _P, _I, _I, _I, ctypes.c_int64, _I, _P]),
    "tl_fp8_absmax_scale": (ctypes.c_int, [_P, _I, ctypes.c_int64, _P, _P]),
    "tl_convert_fp8": (ctypes.c_int, [_P, _P, _I, ctypes.c_int64, _F, _P]),
    "tl_kivi_compressed_bytes": (ctypes.c_size_t, [_I, _I, _I]),
    "tl_kivi_params_supported": (ctypes.c_int, [_I, _I, _I]),
    "tl_kivi_compress": (ctypes.c_int, [_P, _P, _I, _I, _I, _I, _P]),
    "tl_kivi_decompress": (ctypes.c_int, [_P, _P, _I, _I, _I, _I, _P]),
    "tl_kivi_quantized_len": (ctypes.c_int32, [_I, _I]),
    "tl_kivi_page_bytes": (ctypes.c_size_t, [_I]),
    "tl_kivi_build_pages": (ctypes.c_int, [ctypes.POINTER(KiviDesc), _P, _P, _P, _P, _P, _P, _I, _P]),
    "tl_kivi_append": (ctypes.c_int, [ctypes.POINTER(KiviDesc), _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "tl_kivi_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(KiviDesc), _I]),
    "tl_kivi_decode_step": (ctypes.c_int, [ctypes.POINTER(KiviDesc), _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _P, ctypes.c_size_t, _P]),
    "tl_attention_plan": (ctypes.c_int, [_I, _I, _I, ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(ctypes.c_float)]),
    "tl_max_blocks_per_seq": (_I, [_I]),
    "tl_build_block_tables": (ctypes.c_int, [_P, _P, _I, _I, _P]),
    "tl_build_slot_mapping": (ctypes.c_int, [_P, _I, _I, _I, _I, _P]),
    "tl_kivi_pass_params": (ctypes.c_int, [_I, _I, _I, ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "tl_kivi_pass_runs": (_I, [_I, _I, _I, _I, _I, ctypes.c_size_t]),
    "tl_chunked_prefill": (ctypes.c_int, [ctypes.POINTER(PrefillDesc), _P, _P, _P, _P, _P, _P, _P, _I, _I, _P]),
    "tl_kivi_paged_attention_decode": (ctypes.c_int, [ctypes.POINTER(KiviDesc), _P, _P, _P, _P, _P, _P, _P, _P, _I, _P, ctypes.c_size_t, _P]),
    "tl_kivi_rope_step_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(KiviDesc), _I]),
    "tl_kivi_rope_decode_step": (ctypes.c_int, [ctypes.POINTER(KiviDesc)] + [_P] * 7 + [_I, _I] + [_P] * 7
                                 + [_I, _P, ctypes.c_size_t, _P]),
    "tl_kivi_paged_attention_decode_pre_rope": (ctypes.c_int, [ctypes.POINTER(KiviDesc)] + [_P] * 8
                                                + [_I, _P, _P, _I, _I, _P, ctypes.c_size_t, _P]),
    "tl_kivi_decode_step_pre_rope": (ctypes.c_int, [ctypes.POINTER(KiviDesc)] + [_P] * 11
                                     + [_I, _P, _P, _I, _I, _P, ctypes.c_size_t, _P]),
    "tl_paged_attention_decode_step": (ctypes.c_int, [ctypes.POINTER(DecodeDesc)] + [_P] * 9
                                       + [_I, _P, ctypes.c_size_t, _P]),
    "tl_engine_apply_config": (ctypes.c_int, [ctypes.POINTER(DecodeDesc), _I, _I, ctypes.c_char_p]),
    "tl_kivi_apply_config": (ctypes.c_int, [ctypes.POINTER(KiviDesc), _I, _I, ctypes.c_char_p, ctypes.c_char_p, _I]),
}


def _hip_runtimes() -> set:
    try:
        with open("/proc/self/maps") as f:
            return {ln.split()[-1] for ln in f if "libamdhip64" in ln}
    except OSError:
        return set()


ABI_VERSION = 5           # TL_ABI_VERSION of include/tl_attn.h


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build() (make -C truellm-engine_amd)")
    # torch ships its own libamdhip64 with the same SONAME as /opt/rocm's.  Loading
    # torch first makes libtlattn.so bind to that runtime, so torch's allocations and
    # streams and our launches share one HIP runtime.  Importing torch does not
    # initialise the GPU.
    import torch  # noqa: F401
    lib = ctypes.CDLL(LIB_PATH)
    if len(_hip_runtimes()) > 1:
        raise RuntimeError(f"two HIP runtimes loaded in one process: {sorted(_hip_runtimes())}")
    for name, (res, args) in _SIG.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    # the structures above mirror include/tl_attn.h at this version
    if lib.tl_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{LIB_PATH} has C ABI version {lib.tl_abi_version()}, this binding {ABI_VERSION}")
    return lib


lib = _load()


def header_functions() -> list[str]:
    """Names of every function declared in include/*.h."""
    names = []
    for fn in sorted(os.listdir(HEADER_DIR)):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(HEADER_DIR, fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^[A-Za-z_][\w \*]*?\b(tl_\w+)\s*\(", text, flags=re.M)
    return names


def last_error() -> str:
    return lib.tl_last_error_string().decode()


def check(rc: int) -> None:
    if rc != OK:
        raise TLError(rc, last_error())


# ---------------------------------------------------------------------------
# torch helpers (import lazily so ABI tests run without touching the GPU)
# ---------------------------------------------------------------------------

def _torch():
    import torch
    return torch


def dtype_code(t) -> int:
    torch = _torch()
    m = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16, torch.uint8: FP8_E4M3}
    if t.dtype not in m:
        raise TLError(ERR_INVALID_ARGUMENT, f"unsupported tensor dtype {t.dtype}")
    return m[t.dtype]


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream=None):
    torch = _torch()
    s = torch.cuda.current_stream() if stream is None else stream
    return ctypes.c_void_p(s.cuda_stream)


# ---------------------------------------------------------------------------
# Reference operator interface (same names, same argument roles)
# ---------------------------------------------------------------------------

def paged_attention_v1(out, q, k_cache, v_cache, block_tables, seq_lens, num_kv_heads, scale,
                       head_size, block_size, stream=None, gqa_map=GQA_MODULO):
    """paged_attention_v1.cu:177: q/out [S, H, D]; k/v_cache [N, n_kv, D, BS]."""
    S, H = q.shape[0], q.shape[1]
    check(lib.tl_paged_attention_v1(
        _ptr(out), _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(block_tables), _ptr(seq_lens),
        S, H, num_kv_heads, head_size, block_size, block_tables.shape[1], k_cache.shape[0],
        scale, dtype_code(q), gqa_map, _stream(stream)))


def paged_attention_v2(out, exp_sums, max_logits, tmp_out, q, k_cache, v_cache, block_tables,
                       seq_lens, num_kv_heads, scale, head_size, block_size, max_context_len,
                       stream=None, gqa_map=GQA_MODULO, scratch_partitions=None):
    """paged_attention_v2.cu:176: scratch exp_sums/max_logits [S, H, P] fp32,
    tmp_out [S, H, P, D] in q's dtype, P = ceil(max_context_len / (32 * BS)).
    scratch_partitions: the P the scratch was allocated for, when larger
    (tl_paged_attention_v2_capacity)."""
    S, H = q.shape[0], q.shape[1]
    args = [_ptr(out), _ptr(exp_sums), _ptr(max_logits), _ptr(tmp_out), _ptr(q), _ptr(k_cache),
            _ptr(v_cache), _ptr(block_tables), _ptr(seq_lens), S, H, num_kv_heads, head_size,
            block_size, block_tables.shape[1], k_cache.shape[0], scale, dtype_code(q), gqa_map,
            max_context_len]
    if scratch_partitions is None:
        check(lib.tl_paged_attention_v2(*args, _stream(stream)))
    else:
        check(lib.tl_paged_attention_v2_capacity(*args, scratch_partitions, _stream(stream)))


def convert_fp8(out, inp, scale, stream=None, n=None):
    """cache_kernels.cu:286: out (uint8 E4M3 codes) = e4m3(inp * scale), n
    elements (default: all of inp)."""
    n = inp.numel() if n is None else n
    check(lib.tl_convert_fp8(_ptr(out), _ptr(inp), dtype_code(inp), n, scale, _stream(stream)))


def v2_plan(num_seqs, num_heads, num_kv_heads, head_size, block_size, dtype, max_context_len,
            scratch_partitions=None):
    """(partitions, partition_tokens) of tl_paged_attention_v2 (with
    scratch_partitions, of tl_paged_attention_v2_capacity) for a call of
    these sizes."""
    pt = ctypes.c_int32(0)
    if scratch_partitions is None:
        P = lib.tl_paged_attention_v2_partitions(num_seqs, num_heads, num_kv_heads, head_size, block_size, dtype,
                                                 max_context_len, ctypes.byref(pt))
    else:
        P = lib.tl_paged_attention_v2_capacity_partitions(num_seqs, num_heads, num_kv_heads, head_size, block_size,
                                                          dtype, max_context_len, scratch_partitions,
                                                          ctypes.byref(pt))
    if P < 0:
        raise TLError(ERR_INVALID_ARGUMENT, "tl_paged_attention_v2_partitions: sizes refused")
    return P, pt.value


def v2_num_partitions(max_context_len: int, block_size: int) -> int:
    pt = 32 * block_size
    return max(1, (max_context_len + pt - 1) // pt)


def reshape_and_cache(key, value, kv_cache, slot_mapping, stream=None):
    """cache_kernels.cu:202: key/value [T, n_kv, D]; kv_cache [2N, n_kv, D, BS]
    holding the K pool then the V pool."""
    T, n_kv, D = key.shape
    N = kv_cache.shape[0] // 2
    k_cache, v_cache = kv_cache[:N], kv_cache[N:]
    reshape_and_cache_split(key, value, k_cache, v_cache, slot_mapping, stream)


def reshape_and_cache_split(key, value, k_cache, v_cache, slot_mapping, stream=None):
    T, n_kv, D = key.shape
    check(lib.tl_reshape_and_cache(
        _ptr(key), _ptr(value), _ptr(k_cache), _ptr(v_cache), _ptr(slot_mapping), T, n_kv, D,
        k_cache.shape[3], k_cache.shape[0], dtype_code(key), _stream(stream)))


ACT_SILU, ACT_GELU, ACT_GELU_TANH = 0, 1, 2


def rms_norm(out, x, weight, eps, stream=None):
    """layernorm_kernels.cu:149: x / out [T, H]."""
    check(lib.tl_rms_norm(_ptr(out), _ptr(x), _ptr(weight), x.shape[0], x.shape[1], eps, dtype_code(x),
                          _stream(stream)))


def fused_add_rms_norm(out, residual, x, weight, eps, stream=None):
    check(lib.tl_fused_add_rms_norm(_ptr(out), _ptr(residual), _ptr(x), _ptr(weight), x.shape[0], x.shape[1], eps,
                                    dtype_code(x), _stream(stream)))


def layer_norm(out, x, weight, bias, eps, stream=None):
    check(lib.tl_layer_norm(_ptr(out), _ptr(x), _ptr(weight), _ptr(bias), x.shape[0], x.shape[1], eps,
                            dtype_code(x), _stream(stream)))


def act_and_mul(out, gate, up, activation=ACT_SILU, stream=None):
    """activation_kernels.cu:57: out = act(gate) * up, elementwise."""
    check(lib.tl_act_and_mul(_ptr(out), _ptr(gate), _ptr(up), gate.numel(), activation, dtype_code(gate),
                             _stream(stream)))


def vq_encode(kv, book, idx, stream=None):
    """vq_cache.cu:74: idx (uint16 / int16 [n]) = nearest entry of book
    [K, D] for each fp16 row of kv [..., D]."""
    D = book.shape[1]
    check(lib.tl_vq_encode(_ptr(kv), _ptr(book), _ptr(idx), kv.numel() // D, D, book.shape[0], _stream(stream)))


def vq_decode(out, book, idx, stream=None):
    D = book.shape[1]
    check(lib.tl_vq_decode(_ptr(out), _ptr(book), _ptr(idx), out.numel() // D, D, book.shape[0], _stream(stream)))


def vq_kmeans_workspace_bytes(n_samples, codebook_size, head_dim):
    return lib.tl_vq_kmeans_workspace_bytes(n_samples, codebook_size, head_dim)


def vq_kmeans(data, book, n_iterations, workspace, stream=None):
    """codebook_init.cu:100: Lloyd iterations over data [n, D] on book [K, D] in place."""
    D = book.shape[1]
    check(lib.tl_vq_kmeans(_ptr(data), _ptr(book), data.numel() // D, book.shape[0], D, n_iterations,
                           _ptr(workspace), workspace.numel() * workspace.element_size(), _stream(stream)))


ROPE_ADJACENT, ROPE_HALVES = 0, 1


def rope_reshape_and_cache(q, key, value, k_cache, v_cache, slot_mapping, positions, cos_table, sin_table,
                           style=ROPE_ADJACENT, q_out=None, stream=None):
    """RoPE on q (into q_out, default in place) and key, then key/value into
    the pools [N, n_kv, D, BS].  Tables fp32 [max_positions, D/2]."""
    T, n_kv, D = key.shape
    H = 0 if q is None else q.shape[1]
    q_out = q if q_out is None else q_out
    check(lib.tl_rope_reshape_and_cache(
        _ptr(q), _ptr(q_out), _ptr(key), _ptr(value), _ptr(k_cache), _ptr(v_cache), _ptr(slot_mapping),
        _ptr(positions), _ptr(cos_table), _ptr(sin_table), cos_table.shape[0], T, H, n_kv, D,
        k_cache.shape[3], k_cache.shape[0], dtype_code(key), style, _stream(stream)))


def _block_bytes(pool):
    return pool[0].numel() * pool.element_size()


def copy_blocks(k_cache, v_cache, block_mapping, stream=None):
    """cache_kernels.cu:234: block_mapping int32 [P, 2] = {src, dst} on the
    device; block src of each pool is copied to block dst."""
    check(lib.tl_copy_blocks(_ptr(k_cache), _ptr(v_cache), _ptr(block_mapping), block_mapping.shape[0],
                             k_cache.shape[0], _block_bytes(k_cache), _stream(stream)))


def swap_blocks(cache, host_cache, block_mapping, direction, stream=None):
    """cache_kernels.cu:264: whole blocks between a device pool and a pinned
    host tensor; direction 0: device -> host, 1: host -> device."""
    check(lib.tl_swap_blocks(_ptr(cache), _ptr(host_cache), _ptr(block_mapping), block_mapping.shape[0],
                             cache.shape[0], host_cache.shape[0], _block_bytes(cache), direction,
                             _stream(stream)))


def reshape_and_cache_fp8(key, value, k_cache, v_cache, slot_mapping, k_scale, v_scale,
                          stream=None):
    T, n_kv, D = key.shape
    check(lib.tl_reshape_and_cache_fp8(
        _ptr(key), _ptr(value), dtype_code(key), _ptr(k_cache), _ptr(v_cache), _ptr(slot_mapping),
        T, n_kv, D, k_cache.shape[3], k_cache.shape[0], k_scale, v_scale, _stream(stream)))


def fp8_absmax_scale(x, scale_out, stream=None):
    check(lib.tl_fp8_absmax_scale(_ptr(x), dtype_code(x), x.numel(), _ptr(scale_out),
                                  _stream(stream)))


def make_decode_desc(q, k_cache, block_tables, num_kv_heads, scale, *, kv_dtype=None,
                     gqa_map=GQA_GROUPED, partition_tokens=0, k_scale=1.0, v_scale=1.0):
    S, H, D = q.shape
    d = DecodeDesc()
    d.num_seqs, d.num_heads, d.num_kv_heads, d.head_size = S, H, num_kv_heads, D
    d.block_size = k_cache.shape[3]
    d.max_blocks_per_seq = block_tables.shape[1]
    d.num_blocks = k_cache.shape[0]
    d.q_dtype = dtype_code(q)
    d.kv_dtype = dtype_code(k_cache) if kv_dtype is None else kv_dtype
    d.gqa_map = gqa_map
    d.partition_tokens = partition_tokens
    d.scale, d.k_scale, d.v_scale = scale, k_scale, v_scale
    return d


def paged_attention_decode_step(desc: DecodeDesc, out, q, key, value, slot_mapping, k_cache, v_cache, block_tables,
                                seq_lens, max_context_len, workspace=None, stream=None):
    """reshape_and_cache of the step's token, then the decode (seq_lens after the append), in one
    call; slot_mapping[s] is the slot of position seq_lens[s] - 1."""
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(lib.tl_paged_attention_decode_step(
        ctypes.byref(desc), _ptr(out), _ptr(q), _ptr(key), _ptr(value), _ptr(slot_mapping), _ptr(k_cache),
        _ptr(v_cache), _ptr(block_tables), _ptr(seq_lens), max_context_len, _ptr(workspace), ws_bytes,
        _stream(stream)))


def workspace_bytes(desc: DecodeDesc, max_context_len: int) -> int:
    return lib.tl_paged_attention_workspace_bytes(ctypes.byref(desc), max_context_len)


def paged_attention_decode(desc: DecodeDesc, out, q, k_cache, v_cache, block_tables, seq_lens,
                           max_context_len, workspace=None, stream=None):
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(lib.tl_paged_attention_decode(
        ctypes.byref(desc), _ptr(out), _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(block_tables),
        _ptr(seq_lens), max_context_len, _ptr(workspace), ws_bytes, _stream(stream)))


NOALLOC_SCRATCH_BYTES = 32 << 20


def paged_attention_decode_noalloc(desc: DecodeDesc, out, q, k_cache, v_cache, block_tables, seq_lens,
                                   max_context_len, stream=None):
    """tl_paged_attention_decode with the library's own split-K scratch (no allocation)."""
    check(lib.tl_paged_attention_decode_noalloc(
        ctypes.byref(desc), _ptr(out), _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(block_tables),
        _ptr(seq_lens), max_context_len, _stream(stream)))


# ---------------------------------------------------------------------------
# Reference KIVI vector codec (kivi_cache.cuh:32-84): same names and roles
# ---------------------------------------------------------------------------

def kivi_compressed_bytes(head_dim, n_outliers, group_size) -> int:
    return lib.tl_kivi_compressed_bytes(head_dim, n_outliers, group_size)


def kivi_params_supported(head_dim, n_outliers, group_size) -> bool:
    return bool(lib.tl_kivi_params_supported(head_dim, n_outliers, group_size))


def kivi_compress(kv_in, out, n_vecs, head_dim, n_outliers, group_size, stream=None):
    """kv_in fp16 [n_vecs, head_dim] -> out uint8 records."""
    check(lib.tl_kivi_compress(_ptr(kv_in), _ptr(out), n_vecs, head_dim, n_outliers, group_size,
                               _stream(stream)))


def kivi_decompress(rec, kv_out, n_vecs, head_dim, n_outliers, group_size, stream=None):
    check(lib.tl_kivi_decompress(_ptr(rec), _ptr(kv_out), n_vecs, head_dim, n_outliers,
                                 group_size, _stream(stream)))


# ---------------------------------------------------------------------------
# Paged KIVI INT4
# ---------------------------------------------------------------------------

def kivi_quantized_len(seq_len, residual_length) -> int:
    return lib.tl_kivi_quantized_len(seq_len, residual_length)


def make_kivi_desc(q, k_cache, block_tables, page_tables, num_pages, num_kv_heads, scale, *,
                   residual_length=128, gqa_map=GQA_GROUPED, partition_pages=0, bits=4, pre_rope_keys=False,
                   build_ahead=False):
    S, H, D = q.shape
    d = KiviDesc()
    d.bits = bits
    d.pre_rope_keys = int(bool(pre_rope_keys))
    d.build_ahead = int(bool(build_ahead))
    d.num_seqs, d.num_heads, d.num_kv_heads, d.head_size = S, H, num_kv_heads, D
    d.block_size = k_cache.shape[3]
    d.max_blocks_per_seq, d.num_blocks = block_tables.shape[1], k_cache.shape[0]
    d.max_pages_per_seq, d.num_pages = page_tables.shape[1], num_pages
    d.residual_length, d.gqa_map, d.partition_pages = residual_length, gqa_map, partition_pages
    d.scale = scale
    return d


def kivi_build_pages(desc, k_cache, v_cache, block_tables, seq_lens, page_tables, pages,
                     max_context_len, stream=None):
    check(lib.tl_kivi_build_pages(ctypes.byref(desc), _ptr(k_cache), _ptr(v_cache),
                                  _ptr(block_tables), _ptr(seq_lens), _ptr(page_tables),
                                  _ptr(pages), max_context_len, _stream(stream)))


def kivi_append(desc, key, value, k_cache, v_cache, slot_mapping, block_tables, seq_lens,
                page_tables, pages, stream=None):
    check(lib.tl_kivi_append(ctypes.byref(desc), _ptr(key), _ptr(value), _ptr(k_cache),
                             _ptr(v_cache), _ptr(slot_mapping), _ptr(block_tables),
                             _ptr(seq_lens), _ptr(page_tables), _ptr(pages), _stream(stream)))


def kivi_workspace_bytes(desc, max_context_len) -> int:
    return lib.tl_kivi_workspace_bytes(ctypes.byref(desc), max_context_len)


def kivi_decode_step(desc, out, q, key, value, slot_mapping, pages, page_tables, k_cache, v_cache,
                     block_tables, seq_lens, max_context_len, workspace=None, stream=None):
    """kivi_append then kivi_paged_attention_decode (seq_lens after the append) in one call and one
    decode launch; slot_mapping[s] is the pool slot of position seq_lens[s] - 1."""
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(lib.tl_kivi_decode_step(
        ctypes.byref(desc), _ptr(out), _ptr(q), _ptr(key), _ptr(value), _ptr(slot_mapping), _ptr(pages),
        _ptr(page_tables), _ptr(k_cache), _ptr(v_cache), _ptr(block_tables), _ptr(seq_lens), max_context_len,
        _ptr(workspace), ws_bytes, _stream(stream)))


def kivi_rope_step_workspace_bytes(desc, max_context_len) -> int:
    return lib.tl_kivi_rope_step_workspace_bytes(ctypes.byref(desc), max_context_len)


def kivi_rope_decode_step(desc, out, q, key, value, positions, cos_table, sin_table, style, slot_mapping, pages,
                          page_tables, k_cache, v_cache, block_tables, seq_lens, max_context_len, workspace,
                          stream=None):
    """RoPE of q and the new keys at positions[s], then kivi_decode_step on the rotated rows (keys are
    stored and quantised rotated)."""
    ws_bytes = workspace.numel() * workspace.element_size()
    check(lib.tl_kivi_rope_decode_step(
        ctypes.byref(desc), _ptr(out), _ptr(q), _ptr(key), _ptr(value), _ptr(positions), _ptr(cos_table),
        _ptr(sin_table), cos_table.shape[0], style, _ptr(slot_mapping), _ptr(pages), _ptr(page_tables),
        _ptr(k_cache), _ptr(v_cache), _ptr(block_tables), _ptr(seq_lens), max_context_len, _ptr(workspace),
        ws_bytes, _stream(stream)))


def engine_apply_config(desc, block_size=16, use_fp8_kv=False, attention_layout="paged"):
    """CudaEngineConfig's attention knobs onto a decode descriptor (raises TLError for what is not
    built; the descriptor is left as it was then)."""
    lay = None if attention_layout is None else attention_layout.encode()
    check(lib.tl_engine_apply_config(ctypes.byref(desc), block_size, int(bool(use_fp8_kv)), lay))


def kivi_apply_config(desc, bits=8, residual_length=128, key_granularity="per_channel",
                      value_granularity="per_token", pre_rope_keys=False):
    """KiviConfig onto a descriptor (raises TLError for what is not built)."""
    kg = None if key_granularity is None else key_granularity.encode()
    vg = None if value_granularity is None else value_granularity.encode()
    check(lib.tl_kivi_apply_config(ctypes.byref(desc), bits, residual_length, kg, vg, int(bool(pre_rope_keys))))


def kivi_paged_attention_decode_pre_rope(desc, out, q, pages, page_tables, k_cache, v_cache, block_tables,
                                         seq_lens, max_context_len, cos_table, sin_table, style, workspace=None,
                                         stream=None):
    """kivi_paged_attention_decode with the keys held before RoPE: each key rotated at its position
    (token index) as it is scored; q is taken as given."""
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(lib.tl_kivi_paged_attention_decode_pre_rope(
        ctypes.byref(desc), _ptr(out), _ptr(q), _ptr(pages), _ptr(page_tables), _ptr(k_cache),
        _ptr(v_cache), _ptr(block_tables), _ptr(seq_lens), max_context_len, _ptr(cos_table), _ptr(sin_table),
        cos_table.shape[0], style, _ptr(workspace), ws_bytes, _stream(stream)))


def kivi_decode_step_pre_rope(desc, out, q, key, value, slot_mapping, pages, page_tables, k_cache, v_cache,
                              block_tables, seq_lens, max_context_len, cos_table, sin_table, style,
                              workspace=None, stream=None):
    """kivi_decode_step with the keys held before RoPE (stored and quantised unrotated, rotated at
    their positions as they are scored); q is taken as given."""
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(lib.tl_kivi_decode_step_pre_rope(
        ctypes.byref(desc), _ptr(out), _ptr(q), _ptr(key), _ptr(value), _ptr(slot_mapping), _ptr(pages),
        _ptr(page_tables), _ptr(k_cache), _ptr(v_cache), _ptr(block_tables), _ptr(seq_lens), max_context_len,
        _ptr(cos_table), _ptr(sin_table), cos_table.shape[0], style, _ptr(workspace), ws_bytes,
        _stream(stream)))


def kivi_paged_attention_decode(desc, out, q, pages, page_tables, k_cache, v_cache, block_tables,
                                seq_lens, max_context_len, workspace=None, stream=None):
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(lib.tl_kivi_paged_attention_decode(
        ctypes.byref(desc), _ptr(out), _ptr(q), _ptr(pages), _ptr(page_tables), _ptr(k_cache),
        _ptr(v_cache), _ptr(block_tables), _ptr(seq_lens), max_context_len, _ptr(workspace),
        ws_bytes, _stream(stream)))


# ---------------------------------------------------------------------------
# chunked prefill + decode rows (no reference counterpart)
# ---------------------------------------------------------------------------

def make_prefill_desc(q, k_cache, block_tables, num_seqs, num_kv_heads, scale, *,
                      gqa_map=GQA_GROUPED, num_prefill_seqs=0, kv_dtype=None, k_scale=1.0, v_scale=1.0):
    """q [total_q, H, 128]; k_cache [N, n_kv, 128, bs]; block_tables [S, max_blocks].
    num_prefill_seqs > 0 declares sequences 0..n-1 the prefill ones (q_len > 1
    only there), which keeps the decode rows out of the prefill grid.
    kv_dtype FP8_E4M3: a pool of E4M3 codes (uint8) with per-tensor scales."""
    d = PrefillDesc()
    d.num_seqs, d.num_heads, d.num_kv_heads, d.head_size = num_seqs, q.shape[1], num_kv_heads, q.shape[2]
    d.block_size = k_cache.shape[3]
    d.max_blocks_per_seq, d.num_blocks = block_tables.shape[1], k_cache.shape[0]
    d.dtype = dtype_code(q)
    d.gqa_map = gqa_map
    d.num_prefill_seqs = num_prefill_seqs
    d.scale = scale
    d.kv_dtype = d.dtype if kv_dtype is None else kv_dtype
    d.k_scale, d.v_scale = k_scale, v_scale
    return d


def chunked_prefill(desc, out, q, cu_q_lens, k_cache, v_cache, block_tables, seq_lens, max_q_len,
                    stream=None):
    """Causal attention of each sequence's query rows (cu_q_lens) against its
    paged keys 0 .. seq_lens[s] - q_len + i; q_len == 1 rows are decode rows."""
    check(lib.tl_chunked_prefill(ctypes.byref(desc), _ptr(out), _ptr(q), _ptr(cu_q_lens),
                                 _ptr(k_cache), _ptr(v_cache), _ptr(block_tables), _ptr(seq_lens),
                                 q.shape[0], max_q_len, _stream(stream)))


# ---------------------------------------------------------------------------
# host-side helpers of the path's callers (numpy in, numpy out; no GPU)
# ---------------------------------------------------------------------------

def attention_plan(max_context_len, block_size, head_size):
    """cuda_engine.cpp:1138-1160: (use_v2, num_partitions, scale)."""
    v2, P, sc = _I(), _I(), ctypes.c_float()
    check(lib.tl_attention_plan(max_context_len, block_size, head_size, ctypes.byref(v2), ctypes.byref(P),
                                ctypes.byref(sc)))
    return bool(v2.value), P.value, sc.value


def max_blocks_per_seq(num_blocks):
    return lib.tl_max_blocks_per_seq(num_blocks)


def build_block_tables(seq_blocks, max_blocks):
    """cuda_allocator.cpp:231-253 for a batch: rows of block ids padded with -1."""
    import numpy as np
    flat = np.ascontiguousarray(np.concatenate([np.asarray(b, np.int32) for b in seq_blocks])
                                if seq_blocks else np.zeros(0, np.int32), dtype=np.int32)
    offs = np.zeros(len(seq_blocks) + 1, np.int32)
    offs[1:] = np.cumsum([len(b) for b in seq_blocks])
    out = np.empty((len(seq_blocks), max_blocks), np.int32)
    check(lib.tl_build_block_tables(flat.ctypes.data if flat.size else None, offs.ctypes.data, len(seq_blocks),
                                    max_blocks, out.ctypes.data))
    return out


def build_slot_mapping(blocks, block_size, seq_start_pos, num_tokens):
    """cuda_allocator.cpp:255-280."""
    import numpy as np
    b = np.ascontiguousarray(blocks, np.int32)
    out = np.empty(num_tokens, np.int32)
    check(lib.tl_build_slot_mapping(b.ctypes.data if b.size else None, b.size, block_size, seq_start_pos,
                                    num_tokens, out.ctypes.data if num_tokens else None))
    return out


def kivi_pass_params(residual_length, bits, head_dim):
    """kv_compression_pass.cpp:29-66: (n_outliers, group_size, enabled)."""
    o, g, e = _I(), _I(), _I()
    check(lib.tl_kivi_pass_params(residual_length, bits, head_dim, ctypes.byref(o), ctypes.byref(g),
                                  ctypes.byref(e)))
    return o.value, g.value, bool(e.value)


def kivi_pass_runs(seq_len, n_kv_heads, head_dim, n_outliers, group_size, scratch_bytes):
    """kv_compression_pass.cpp:184-216: does run_kivi compress this layer?"""
    return bool(lib.tl_kivi_pass_runs(seq_len, n_kv_heads, head_dim, n_outliers, group_size, scratch_bytes))
