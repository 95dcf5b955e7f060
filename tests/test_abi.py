"""C ABI checks that need no GPU: the library loads, exports every function
include/*.h declares, and rejects bad calls with an error code before any
HIP call is made."""
import ctypes

import pytest

import tl_attn as tla


def test_exports_every_declared_function():
    names = tla.header_functions()
    assert len(names) >= 9
    missing = [n for n in names if not hasattr(tla.lib, n)]
    assert not missing, missing


def test_abi_version():
    assert tla.lib.tl_abi_version() == 5 == tla.ABI_VERSION


def _desc(**kw):
    d = tla.DecodeDesc()
    d.num_seqs, d.num_heads, d.num_kv_heads, d.head_size, d.block_size = 4, 32, 8, 128, 16
    d.max_blocks_per_seq, d.num_blocks = 64, 512
    d.q_dtype = d.kv_dtype = tla.F16
    d.gqa_map, d.partition_tokens = tla.GQA_GROUPED, 0
    d.scale, d.k_scale, d.v_scale = 0.088, 1.0, 1.0
    for k, v in kw.items():
        setattr(d, k, v)
    return d


FAKE = ctypes.c_void_p(0x1000)  # never dereferenced: every call below fails validation


def _decode(d, out=FAKE, ws=None, ws_bytes=0, max_ctx=1024):
    return tla.lib.tl_paged_attention_decode(ctypes.byref(d), out, FAKE, FAKE, FAKE, FAKE, FAKE,
                                             max_ctx, ws, ws_bytes, None)


@pytest.mark.parametrize("kw,code", [
    (dict(num_heads=30), tla.ERR_INVALID_ARGUMENT),
    (dict(num_kv_heads=0), tla.ERR_INVALID_ARGUMENT),
    (dict(head_size=72), tla.ERR_NOT_IMPLEMENTED),
    (dict(head_size=80, block_size=32), tla.ERR_NOT_IMPLEMENTED),
    (dict(head_size=80, kv_dtype=tla.FP8_E4M3), tla.ERR_NOT_IMPLEMENTED),
    (dict(head_size=64, block_size=8), tla.ERR_NOT_IMPLEMENTED),
    (dict(block_size=12), tla.ERR_NOT_IMPLEMENTED),
    (dict(block_size=512), tla.ERR_NOT_IMPLEMENTED),
    (dict(block_size=32, q_dtype=tla.F32, kv_dtype=tla.F32), tla.ERR_NOT_IMPLEMENTED),
    (dict(q_dtype=7), tla.ERR_INVALID_ARGUMENT),
    (dict(kv_dtype=tla.BF16), tla.ERR_NOT_IMPLEMENTED),
    (dict(kv_dtype=tla.FP8_E4M3, q_dtype=tla.F32), tla.ERR_NOT_IMPLEMENTED),
    (dict(gqa_map=5), tla.ERR_INVALID_ARGUMENT),
    (dict(partition_tokens=100), tla.ERR_INVALID_ARGUMENT),
    (dict(num_blocks=0), tla.ERR_INVALID_ARGUMENT),
])
def test_decode_rejects_bad_descriptors(kw, code):
    assert _decode(_desc(**kw)) == code
    assert tla.last_error()


@pytest.mark.parametrize("kw", [
    dict(block_size=8), dict(block_size=32), dict(block_size=64), dict(block_size=128),
    dict(block_size=256), dict(block_size=16, kv_dtype=tla.FP8_E4M3), dict(block_size=8, kv_dtype=tla.FP8_E4M3),
    dict(block_size=256, kv_dtype=tla.FP8_E4M3, q_dtype=tla.BF16), dict(head_size=80), dict(head_size=96),
    dict(head_size=96, q_dtype=tla.BF16, kv_dtype=tla.BF16), dict(head_size=64, q_dtype=tla.F32, kv_dtype=tla.F32),
    dict(head_size=256, q_dtype=tla.F32, kv_dtype=tla.F32), dict(head_size=256, kv_dtype=tla.FP8_E4M3),
])
def test_decode_accepts_the_built_shapes(kw):
    """Head 128 with any power-of-two block size 8..256 (FP8 too), the
    reference's F16 heads 64/80/96/256 and F32 heads 64/128/256 at block
    size 16 (paged_attention_v1.cu:198-209): validation passes, so the
    split-K plan has a workspace size."""
    d = _desc(partition_tokens=512, **kw)
    assert tla.workspace_bytes(d, 4096) == 4 * 32 * 8 * (d.head_size * 4 + 8), tla.last_error()


def test_decode_rejects_null_and_missing_workspace():
    assert tla.lib.tl_paged_attention_decode(None, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 10, None, 0,
                                             None) == tla.ERR_INVALID_ARGUMENT
    assert _decode(_desc(), out=None) == tla.ERR_INVALID_ARGUMENT
    d = _desc(partition_tokens=512)
    need = tla.workspace_bytes(d, 4096)
    assert need == 4 * 32 * 8 * (128 * 4 + 8)
    assert _decode(d, max_ctx=4096) == tla.ERR_INVALID_ARGUMENT
    assert "workspace" in tla.last_error()


def test_workspace_is_zero_for_single_pass():
    assert tla.workspace_bytes(_desc(partition_tokens=-1), 32768) == 0
    assert tla.workspace_bytes(_desc(), 512) == 0


def test_auto_partitioning_targets_many_workgroups():
    # 64 x 8 work items already fill the GPU: single pass
    assert tla.workspace_bytes(_desc(num_seqs=64), 4096) == 0
    # 4 x 8 items at 4096 tokens -> 8 partitions of 512
    assert tla.workspace_bytes(_desc(num_seqs=4), 4096) == 4 * 32 * 8 * (128 * 4 + 8)
    # 16 x 8 items at 32768 tokens -> 4 partitions of 8192
    assert tla.workspace_bytes(_desc(num_seqs=16), 32768) == 16 * 32 * 4 * (128 * 4 + 8)
    # fewer items than CUs even at 512 tokens (the engine's one-sequence
    # call): partitions down to one iteration per wavefront of a 4-wavefront
    # workgroup, so that about 256 workgroups share the context
    assert tla.workspace_bytes(_desc(num_seqs=1), 4096) == 1 * 32 * 32 * (128 * 4 + 8)    # 32 x 128
    assert tla.workspace_bytes(_desc(num_seqs=2), 4096) == 2 * 32 * 16 * (128 * 4 + 8)    # 16 x 256
    assert tla.workspace_bytes(_desc(num_seqs=1, kv_dtype=tla.FP8_E4M3), 4096) == 32 * 16 * (128 * 4 + 8)
    assert tla.workspace_bytes(_desc(num_seqs=1), 1024) == 32 * 8 * (128 * 4 + 8)         # 8 x 128
    # 49 partitions of 2048 tokens already give 392 workgroups
    assert tla.workspace_bytes(_desc(num_seqs=1), 100000) == 32 * 49 * (128 * 4 + 8)
    assert tla.workspace_bytes(_desc(num_seqs=1), 512) == 0                              # single pass
    # the dot-product decode (head 80) keeps kDecodeChunk partitions
    assert tla.workspace_bytes(_desc(num_seqs=1, head_size=80), 4096) == 32 * 8 * (80 * 4 + 8)


def test_v2_plan_inside_the_callers_scratch():
    """tl_paged_attention_v2's plan: f16 at head 128 keeps f16 partials, one
    partition per reference-kernel slot ((max_ctx / bs + 31) / 32); bf16 and
    f32 keep fp32 partials (half as many for bf16); a batch that fills the
    GPU runs single pass."""
    plan = lambda S, dt, L, bs=16, hs=128: tla.v2_plan(S, 32, 8, hs, bs, dt, L)
    assert plan(1, tla.F16, 4096) == (8, 512)           # the engine's call: 8 slots, the plan wants 32
    assert plan(1, tla.BF16, 4096) == (4, 1024)         # fp32 partials: 4 of the 8 slots' bytes
    assert plan(1, tla.F32, 4096) == (8, 512)
    assert plan(1, tla.F16, 1541) == (3, 640)           # kernel count 3 (the engine's is 4)
    assert plan(1, tla.F16, 600) == (2, 384)
    assert plan(64, tla.F16, 4096) == (1, 0)            # single pass
    assert plan(4, tla.F16, 4096) == (8, 512)           # the library plan fits
    assert plan(1, tla.F16, 4096, hs=80)[0] == 4        # dot-product decode: fp32 partials
    with pytest.raises(tla.TLError):
        plan(1, tla.F16, 4096, bs=12)


def test_v2_capacity_plan_uses_the_callers_allocation():
    """tl_paged_attention_v2_capacity: a scratch allocated for more
    partitions than the call's context needs (the engine's, sized for its
    training context) lets the one-sequence plan take shorter partitions;
    a count below the reference kernel's for the call is refused."""
    plan = lambda S, dt, L, cap: tla.v2_plan(S, 32, 8, 128, 16, dt, L, scratch_partitions=cap)
    assert plan(1, tla.F16, 4096, 8) == (8, 512)          # as tl_paged_attention_v2
    assert plan(1, tla.F16, 4096, 16) == (16, 256)        # n_ctx_train 8192: 16 slots
    assert plan(1, tla.F16, 4096, 64) == (32, 128)        # the library plan fits
    assert plan(1, tla.BF16, 4096, 16) == (8, 512)        # fp32 partials: 8 of the 16 slots' bytes
    assert plan(64, tla.F16, 4096, 16) == (1, 0)          # single pass
    with pytest.raises(tla.TLError):
        plan(1, tla.F16, 4096, 7)                           # below the 8 the call needs
    with pytest.raises(tla.TLError):
        plan(1, tla.F16, 4096, 0)
    call = lambda cap: tla.lib.tl_paged_attention_v2_capacity(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                                                              1, 32, 8, 128, 16, 256, 512, 0.088, tla.F16,
                                                              tla.GQA_GROUPED, 4096, cap, None)
    assert call(7) == tla.ERR_INVALID_ARGUMENT and "scratch_partitions" in tla.last_error()
    assert call(0) == tla.ERR_INVALID_ARGUMENT


@pytest.mark.parametrize("kw,ok", [
    (dict(partition_tokens=96), True), (dict(partition_tokens=32), True),
    (dict(partition_tokens=96, kv_dtype=tla.FP8_E4M3), False), (dict(partition_tokens=192, kv_dtype=tla.FP8_E4M3), True),
    (dict(partition_tokens=1024, head_size=80), True), (dict(partition_tokens=256, head_size=80), False),
])
def test_partition_tokens_granularity(kw, ok):
    """Explicit partitions: a multiple of the matrix-core wavefront's
    iteration (32 tokens of 2-byte KV, 64 of FP8) at head 128, of 512 for
    the other kernels."""
    d = _desc(**kw)
    got = tla.workspace_bytes(d, 4096)
    if ok:
        P = -(-4096 // d.partition_tokens)
        assert got == 4 * 32 * P * (d.head_size * 4 + 8)
    else:
        assert got == 0 and _decode(d, max_ctx=4096) == tla.ERR_INVALID_ARGUMENT


def test_empty_batch_is_a_no_op():
    d = _desc(num_seqs=0)
    assert tla.lib.tl_paged_attention_decode(ctypes.byref(d), None, None, None, None, None, None,
                                             0, None, 0, None) == tla.OK
    assert tla.lib.tl_reshape_and_cache(None, None, None, None, None, 0, 8, 128, 16, 10,
                                        tla.F16, None) == tla.OK


def test_v1_v2_reject_like_decode():
    rc = tla.lib.tl_paged_attention_v1(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4, 32, 8, 72, 16, 64,
                                       512, 0.1, tla.F16, 0, None)
    assert rc == tla.ERR_NOT_IMPLEMENTED
    rc = tla.lib.tl_paged_attention_v2(FAKE, None, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4, 32,
                                       8, 128, 16, 64, 512, 0.1, tla.F16, 0, 4096, None)
    assert rc == tla.ERR_INVALID_ARGUMENT
    # misaligned pool
    rc = tla.lib.tl_paged_attention_v1(FAKE, FAKE, ctypes.c_void_p(0x1002), FAKE, FAKE, FAKE, 4,
                                       32, 8, 128, 16, 64, 512, 0.1, tla.F16, 0, None)
    assert rc == tla.ERR_INVALID_ARGUMENT


def test_convert_fp8_rejects_bad_arguments():
    L = tla.lib
    L.tl_convert_fp8.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float,
                                 ctypes.c_void_p]
    assert L.tl_convert_fp8(FAKE, FAKE, tla.F16, -1, 1.0, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_convert_fp8(FAKE, FAKE, tla.FP8_E4M3, 16, 1.0, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_convert_fp8(None, FAKE, tla.F16, 16, 1.0, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_convert_fp8(FAKE, ctypes.c_void_p(0x1001), tla.F16, 16, 1.0, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_convert_fp8(FAKE, ctypes.c_void_p(0x1002), tla.F32, 16, 1.0, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_convert_fp8(None, None, tla.F16, 0, 1.0, None) == tla.OK


def test_reshape_rejects_bad_arguments():
    L = tla.lib
    assert L.tl_reshape_and_cache(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 8, 100, 16, 10, tla.F16,
                                  None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_reshape_and_cache(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 8, 128, 16, 10, 9,
                                  None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_reshape_and_cache(None, FAKE, FAKE, FAKE, FAKE, 4, 8, 128, 16, 10, tla.F16,
                                  None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_reshape_and_cache_fp8(FAKE, FAKE, tla.F32, FAKE, FAKE, FAKE, 4, 8, 128, 16, 10,
                                      1.0, 1.0, None) == tla.ERR_NOT_IMPLEMENTED
    assert L.tl_fp8_absmax_scale(FAKE, tla.F16, -1, FAKE, None) == tla.ERR_INVALID_ARGUMENT


def test_block_ops_reject_bad_arguments_and_empty_is_a_no_op():
    L = tla.lib
    assert L.tl_copy_blocks(FAKE, FAKE, FAKE, 3, 0, 4096, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_copy_blocks(FAKE, FAKE, FAKE, -1, 8, 4096, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_copy_blocks(FAKE, FAKE, FAKE, 3, 8, 0, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_copy_blocks(None, FAKE, FAKE, 3, 8, 4096, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_copy_blocks(None, None, None, 0, 8, 4096, None) == tla.OK
    assert L.tl_swap_blocks(FAKE, FAKE, FAKE, 3, 8, 8, 4096, 2, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_swap_blocks(FAKE, FAKE, FAKE, 3, 8, 0, 4096, 0, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_swap_blocks(FAKE, None, FAKE, 3, 8, 8, 4096, 1, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_swap_blocks(None, None, None, 0, 8, 8, 4096, 0, None) == tla.OK


def test_rope_rejects_bad_arguments():
    L = tla.lib
    args = lambda **kw: [kw.get(k, v) for k, v in [
        ("q", FAKE), ("q_out", FAKE), ("key", FAKE), ("value", FAKE), ("kc", FAKE), ("vc", FAKE),
        ("slots", FAKE), ("pos", FAKE), ("cos", FAKE), ("sin", FAKE), ("max_pos", 4096), ("T", 4), ("H", 32),
        ("n_kv", 8), ("D", 128), ("BS", 16), ("N", 64), ("dtype", tla.F16), ("style", 0), ("stream", None)]]
    f = L.tl_rope_reshape_and_cache
    assert f(*args(D=120)) == tla.ERR_INVALID_ARGUMENT
    assert f(*args(style=2)) == tla.ERR_INVALID_ARGUMENT
    assert f(*args(dtype=9)) == tla.ERR_INVALID_ARGUMENT
    assert f(*args(max_pos=0)) == tla.ERR_INVALID_ARGUMENT
    assert f(*args(cos=None)) == tla.ERR_INVALID_ARGUMENT
    assert f(*args(q=None)) == tla.ERR_INVALID_ARGUMENT
    assert f(*args(T=0, q=None, key=None)) == tla.OK


def test_vq_rejects_bad_arguments():
    L = tla.lib
    assert L.tl_vq_encode(FAKE, FAKE, FAKE, 4, 12, 256, None) == tla.ERR_INVALID_ARGUMENT     # head_dim % 8
    assert L.tl_vq_encode(FAKE, FAKE, FAKE, 4, 264, 256, None) == tla.ERR_INVALID_ARGUMENT    # > 256
    assert L.tl_vq_encode(FAKE, FAKE, FAKE, 4, 128, 0, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_vq_encode(FAKE, FAKE, FAKE, 4, 128, 65537, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_vq_encode(FAKE, ctypes.c_void_p(0x1002), FAKE, 4, 128, 256, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_vq_decode(None, FAKE, FAKE, 4, 128, 256, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_vq_encode(None, None, None, 0, 128, 256, None) == tla.OK
    need = L.tl_vq_kmeans_workspace_bytes(1000, 256, 128)
    assert need >= 1000 * 4 + 256 * 128 * 12
    assert L.tl_vq_kmeans(FAKE, FAKE, 1000, 256, 128, 5, FAKE, need - 1, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_vq_kmeans(FAKE, FAKE, 1000, 256, 128, -1, FAKE, need, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_vq_kmeans(FAKE, FAKE, 1000, 256, 128, 0, FAKE, need, None) == tla.OK


def test_norm_act_reject_bad_arguments():
    L = tla.lib
    assert L.tl_rms_norm(FAKE, FAKE, FAKE, 4, 0, 1e-5, tla.F16, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_rms_norm(FAKE, FAKE, FAKE, 4, 128, 1e-5, 9, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_rms_norm(None, FAKE, FAKE, 4, 128, 1e-5, tla.F16, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_fused_add_rms_norm(FAKE, None, FAKE, FAKE, 4, 128, 1e-5, tla.F16, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_layer_norm(FAKE, FAKE, FAKE, None, 4, 128, 1e-5, tla.F16, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_act_and_mul(FAKE, FAKE, FAKE, 16, 3, tla.F16, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_act_and_mul(FAKE, FAKE, FAKE, -1, 0, tla.F16, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_act_and_mul(None, None, None, 0, 0, tla.F16, None) == tla.OK
    assert L.tl_rms_norm(None, None, None, 0, 128, 1e-5, tla.F16, None) == tla.OK


def test_kivi_host_helpers_match_reference_known_answers():
    # test_kivi_bounds.cpp:25-69, through the library
    assert tla.kivi_compressed_bytes(128, 8, 16) == 24 + 8 * 12
    assert tla.kivi_compressed_bytes(64, 0, 16) == 4 * 12
    assert tla.kivi_compressed_bytes(64, 64, 16) == 64 * 3
    assert tla.kivi_params_supported(128, 8, 16)
    assert tla.kivi_params_supported(64, 4, 16)
    assert tla.kivi_params_supported(tla.KIVI_MAX_HEAD_DIM, tla.KIVI_MAX_OUTLIERS, 16)
    for bad in [(129, 8, 16), (128, 65, 16), (16, 32, 16), (128, 8, 0), (128, 8, -4), (0, 0, 16),
                (-1, 0, 16)]:
        assert not tla.kivi_params_supported(*bad)
    assert tla.KIVI_MAX_HEAD_DIM == 128 and tla.KIVI_MAX_OUTLIERS == 64


def test_kivi_quantized_len():
    assert tla.kivi_quantized_len(4096, 128) == 3968
    assert tla.kivi_quantized_len(159, 128) == 0
    assert tla.kivi_quantized_len(160, 128) == 32
    assert tla.kivi_quantized_len(5, 0) == 0 and tla.kivi_quantized_len(64, 0) == 64


def test_kivi_codec_rejects_unsupported_and_odd_groups():
    L = tla.lib
    assert L.tl_kivi_compress(FAKE, FAKE, 1, 256, 0, 16, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_kivi_compress(FAKE, FAKE, 1, 128, 8, 5, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_kivi_decompress(FAKE, FAKE, -1, 128, 8, 16, None) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_kivi_compress(None, None, 0, 128, 8, 16, None) == tla.OK


def _kdesc(**kw):
    d = tla.KiviDesc()
    d.num_seqs, d.num_heads, d.num_kv_heads, d.head_size, d.block_size = 64, 32, 8, 128, 16
    d.max_blocks_per_seq, d.num_blocks, d.max_pages_per_seq, d.num_pages = 256, 20480, 128, 8192
    d.residual_length, d.gqa_map, d.partition_pages, d.scale = 128, 1, 0, 0.088
    for k, v in kw.items():
        setattr(d, k, v)
    return d


def test_kivi_decode_descriptor_checks_and_planning():
    L = tla.lib
    call = lambda d: L.tl_kivi_paged_attention_decode(ctypes.byref(d), FAKE, FAKE, FAKE, FAKE,
                                                      FAKE, FAKE, FAKE, FAKE, 4096, None, 0, None)
    assert call(_kdesc(head_size=64)) == tla.ERR_NOT_IMPLEMENTED
    # the fp16 pool's block size: any power of two 8..256 (CudaEngineConfig's
    # paged_kv_block_size, config_schema.h:68); the checks pass and the call
    # fails later on its missing workspace
    for bs in (12, 4, 512, 0):
        assert call(_kdesc(block_size=bs)) == tla.ERR_NOT_IMPLEMENTED
    for bs in (8, 32, 64, 256):
        assert tla.kivi_workspace_bytes(_kdesc(num_seqs=4, block_size=bs), 4096) == 4 * 32 * 16 * (128 * 4 + 8)
        assert call(_kdesc(num_seqs=4, block_size=bs)) == tla.ERR_INVALID_ARGUMENT
    assert call(_kdesc(residual_length=-1)) == tla.ERR_INVALID_ARGUMENT
    assert call(_kdesc(num_pages=0)) == tla.ERR_INVALID_ARGUMENT
    assert tla.kivi_workspace_bytes(_kdesc(), 4096) == 0               # 512 items: single pass
    # 4 x 8 items, 124 pages -> 16 partitions of 8 pages
    assert tla.kivi_workspace_bytes(_kdesc(num_seqs=4), 4096) == 4 * 32 * 16 * (128 * 4 + 8)
    assert call(_kdesc(num_seqs=4)) == tla.ERR_INVALID_ARGUMENT        # workspace missing
    # page code widths: 4 (also 0) and 8; at 4096 tokens the workspace does
    # not depend on them
    assert call(_kdesc(bits=5)) == tla.ERR_NOT_IMPLEMENTED
    assert call(_kdesc(bits=2)) == tla.ERR_NOT_IMPLEMENTED
    assert tla.kivi_workspace_bytes(_kdesc(num_seqs=4, bits=8), 4096) == 4 * 32 * 16 * (128 * 4 + 8)
    # the _pre_rope entry points give a workgroup at most 160 (INT4) / 144
    # (INT8) pages, their rotations held in LDS: the 300 pages of 9728 tokens
    # run in 2 / 3 partitions, a single pass asked for included, and the
    # workspace is sized for that plan
    for pp in (0, -1):
        assert tla.kivi_workspace_bytes(_kdesc(partition_pages=pp), 9728) == 64 * 32 * 2 * (128 * 4 + 8)
        assert tla.kivi_workspace_bytes(_kdesc(partition_pages=pp, bits=8), 9728) == 64 * 32 * 3 * (128 * 4 + 8)
    assert tla.kivi_workspace_bytes(_kdesc(partition_pages=-1), 4096) == 0
    # build_ahead: 0 or 1 (with any residual length: below 9 it builds on completion)
    for ba in (2, -1):
        assert call(_kdesc(build_ahead=ba)) == tla.ERR_INVALID_ARGUMENT
    for ba, R in ((1, 128), (1, 4), (0, 128)):
        assert call(_kdesc(num_seqs=4, build_ahead=ba, residual_length=R)) == tla.ERR_INVALID_ARGUMENT  # workspace
    assert ctypes.sizeof(tla.KiviDesc) == 16 * 4


def test_kivi_page_bytes():
    assert tla.kivi_page_bytes(4) == tla.KIVI_PAGE_BYTES == 5120
    assert tla.kivi_page_bytes(0) == 5120
    assert tla.kivi_page_bytes(8) == tla.KIVI_PAGE_BYTES_INT8 == 9216
    assert tla.kivi_page_bytes(3) == 0 and tla.kivi_page_bytes(16) == 0


def test_chunked_prefill_argument_checks():
    """tl_chunked_prefill: the arguments its kernels assume, checked before
    any device work (out 4-byte aligned: the epilogue stores two channels per
    4-byte store; max_q_len x group below 2^22 - 256: the kernel's
    row -> (query, head) map is exact only there)."""
    L = tla.lib
    def desc(**kw):
        d = tla.PrefillDesc()
        d.num_seqs, d.num_heads, d.num_kv_heads, d.head_size, d.block_size = 2, 32, 8, 128, 16
        d.max_blocks_per_seq, d.num_blocks, d.dtype, d.gqa_map, d.num_prefill_seqs = 64, 256, tla.BF16, 1, 0
        d.scale = 0.088
        for k, v in kw.items():
            setattr(d, k, v)
        return d
    def call(d, out=FAKE, total_q=1024, max_q=512):
        return L.tl_chunked_prefill(ctypes.byref(d), out, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, total_q, max_q, None)
    assert call(desc(), out=ctypes.c_void_p(0x1002)) == tla.ERR_INVALID_ARGUMENT
    assert "4-byte" in tla.last_error()
    big = (1 << 22) // 4                       # group 4: max_q_len x 4 reaches 2^22
    assert call(desc(), total_q=big, max_q=big) == tla.ERR_NOT_IMPLEMENTED
    assert call(desc(dtype=tla.F32)) == tla.ERR_NOT_IMPLEMENTED
    assert call(desc(head_size=64)) == tla.ERR_NOT_IMPLEMENTED
    # the pool: the q type or FP8 E4M3 (positive finite scales), any
    # power-of-two block size 8..256; the checks before the pointer checks
    assert call(desc(kv_dtype=tla.F16)) == tla.ERR_NOT_IMPLEMENTED   # bf16 q over an f16 pool
    assert call(desc(kv_dtype=tla.FP8_E4M3, k_scale=0.0, v_scale=1.0)) == tla.ERR_INVALID_ARGUMENT
    assert call(desc(kv_dtype=tla.FP8_E4M3, k_scale=1.0, v_scale=float("inf"))) == tla.ERR_INVALID_ARGUMENT
    for bs in (4, 12, 512):
        assert call(desc(block_size=bs)) == tla.ERR_NOT_IMPLEMENTED
    for bs in (8, 16, 32, 64, 128, 256):
        for kw in (dict(), dict(kv_dtype=tla.FP8_E4M3, k_scale=0.5, v_scale=2.0)):
            assert call(desc(block_size=bs, **kw), out=None) == tla.ERR_INVALID_ARGUMENT   # NULL out: checks passed
            assert "NULL" in tla.last_error()
    assert call(desc(), max_q=2048) == tla.ERR_INVALID_ARGUMENT      # max_q_len > total_q
    assert call(desc(scale=0.0)) == tla.ERR_INVALID_ARGUMENT


def test_decode_step_argument_checks():
    """tl_paged_attention_decode_step checks the decode's arguments and its
    own (the token's rows and slots) before any device work."""
    L = tla.lib
    d = _desc()
    def call(key=FAKE, value=FAKE, slots=FAKE, desc=d):
        return L.tl_paged_attention_decode_step(ctypes.byref(desc), FAKE, FAKE, key, value, slots, FAKE, FAKE, FAKE,
                                                FAKE, 1024, FAKE, 1 << 30, None)
    assert call(key=None) == tla.ERR_INVALID_ARGUMENT
    assert call(value=None) == tla.ERR_INVALID_ARGUMENT
    assert call(slots=None) == tla.ERR_INVALID_ARGUMENT
    assert call(key=ctypes.c_void_p(0x1008)) == tla.ERR_INVALID_ARGUMENT      # not 16-byte aligned
    assert call(desc=_desc(head_size=100)) == tla.ERR_NOT_IMPLEMENTED
    assert call(key=None, desc=_desc(num_seqs=0)) == tla.OK


def test_engine_apply_config_maps_cudaengineconfig():
    """CudaEngineConfig (config_schema.h:67-83): paged_kv_block_size, use_fp8_kv
    and attention_layout onto a decode descriptor.  Both layouts name the
    [N, n_kv, d, bs] pool; a rejected call leaves the descriptor as it was."""
    d = _desc(q_dtype=tla.BF16, kv_dtype=tla.BF16)
    tla.engine_apply_config(d, block_size=32)
    assert d.block_size == 32 and d.kv_dtype == tla.BF16
    d.k_scale = d.v_scale = 0.0
    tla.engine_apply_config(d, block_size=16, use_fp8_kv=True, attention_layout="flash_paged")
    assert d.block_size == 16 and d.kv_dtype == tla.FP8_E4M3 and d.k_scale == 1.0 and d.v_scale == 1.0
    tla.engine_apply_config(d, block_size=64, use_fp8_kv=False)
    assert d.block_size == 64 and d.kv_dtype == tla.BF16
    L = tla.lib
    call = lambda bs, fp8, lay: L.tl_engine_apply_config(ctypes.byref(d), bs, fp8, lay)
    assert call(48, 0, b"paged") == tla.ERR_INVALID_ARGUMENT           # not a power of two
    assert call(0, 0, b"paged") == tla.ERR_INVALID_ARGUMENT
    assert call(16, 0, b"flash") == tla.ERR_NOT_IMPLEMENTED
    assert "attention_layout" in tla.last_error()
    assert call(16, 0, None) == tla.ERR_NOT_IMPLEMENTED
    assert call(512, 0, b"paged") == tla.ERR_NOT_IMPLEMENTED           # no kernel for block size 512
    assert L.tl_engine_apply_config(None, 16, 0, b"paged") == tla.ERR_INVALID_ARGUMENT
    assert d.block_size == 64 and d.kv_dtype == tla.BF16              # unchanged by the rejected calls
    tla.engine_apply_config(d, block_size=8, use_fp8_kv=True)           # every power of two 8..256, FP8 too
    assert d.block_size == 8 and d.kv_dtype == tla.FP8_E4M3
    tla.engine_apply_config(d, block_size=64, use_fp8_kv=False)
    f32 = _desc(q_dtype=tla.F32, kv_dtype=tla.F32)
    assert L.tl_engine_apply_config(ctypes.byref(f32), 16, 1, b"paged") == tla.ERR_NOT_IMPLEMENTED  # FP8 needs 2-byte q


def test_kivi_apply_config_maps_kiviconfig_and_rejects_what_is_not_built():
    """KiviConfig (config_schema.h:122-129): bits, residual_length and
    pre_rope_keys land in the descriptor; the default granularities are the
    pages' layout; other granularities are not built."""
    d = _kdesc(bits=0, residual_length=5)
    tla.kivi_apply_config(d, bits=8, residual_length=128)
    assert d.bits == 8 and d.residual_length == 128 and d.pre_rope_keys == 0
    tla.kivi_apply_config(d, bits=4, residual_length=0, pre_rope_keys=True)
    assert d.bits == 4 and d.residual_length == 0 and d.pre_rope_keys == 1
    L = tla.lib
    call = lambda b, r, kg, vg, pre: L.tl_kivi_apply_config(ctypes.byref(d), b, r, kg, vg, pre)
    assert call(8, 128, b"per_channel", b"per_token", 2) == tla.ERR_INVALID_ARGUMENT
    assert "pre_rope_keys" in tla.last_error()
    assert call(8, 128, b"per_token", b"per_token", 0) == tla.ERR_NOT_IMPLEMENTED
    assert call(8, 128, b"per_channel", b"per_channel", 0) == tla.ERR_NOT_IMPLEMENTED
    assert call(8, 128, None, b"per_token", 0) == tla.ERR_NOT_IMPLEMENTED
    assert call(6, 128, b"per_channel", b"per_token", 0) == tla.ERR_INVALID_ARGUMENT
    assert call(8, -1, b"per_channel", b"per_token", 0) == tla.ERR_INVALID_ARGUMENT
    assert L.tl_kivi_apply_config(None, 8, 128, b"per_channel", b"per_token", 0) == tla.ERR_INVALID_ARGUMENT
    # a rejected call leaves the descriptor
    assert d.bits == 4 and d.residual_length == 0 and d.pre_rope_keys == 1


def test_kivi_pre_rope_entry_points_check_their_arguments():
    """Keys held before RoPE: the standard decode and step refuse a
    descriptor with pre_rope_keys set (they would score unrotated keys); the
    _pre_rope entry points check the tables (non-NULL, 16-byte aligned,
    max_positions > 0 and covering max_context_len, style 0 or 1) before any
    device work."""
    L = tla.lib
    d = _kdesc()
    d.pre_rope_keys = 1
    assert L.tl_kivi_paged_attention_decode(ctypes.byref(d), FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                                            4096, FAKE, 1 << 30, None) == tla.ERR_INVALID_ARGUMENT
    assert "pre_rope_keys" in tla.last_error()
    assert L.tl_kivi_decode_step(ctypes.byref(d), *([FAKE] * 11), 4096, FAKE, 1 << 30, None) == tla.ERR_INVALID_ARGUMENT
    d.pre_rope_keys = 3
    assert L.tl_kivi_paged_attention_decode_pre_rope(ctypes.byref(d), *([FAKE] * 8), 4096, FAKE, FAKE, 8192, 0, FAKE,
                                                     1 << 30, None) == tla.ERR_INVALID_ARGUMENT
    d.pre_rope_keys = 1

    def dec(cos=FAKE, sin=FAKE, max_pos=8192, style=0):
        return L.tl_kivi_paged_attention_decode_pre_rope(ctypes.byref(d), *([FAKE] * 8), 4096, cos, sin, max_pos,
                                                         style, FAKE, 1 << 30, None)

    def step(cos=FAKE, sin=FAKE, max_pos=8192, style=1):
        return L.tl_kivi_decode_step_pre_rope(ctypes.byref(d), *([FAKE] * 11), 4096, cos, sin, max_pos, style, FAKE,
                                              1 << 30, None)
    for f in (dec, step):
        assert f(cos=None) == tla.ERR_INVALID_ARGUMENT
        assert f(sin=None) == tla.ERR_INVALID_ARGUMENT
        assert f(cos=ctypes.c_void_p(0x1004)) == tla.ERR_INVALID_ARGUMENT
        assert "aligned" in tla.last_error()
        assert f(max_pos=0) == tla.ERR_INVALID_ARGUMENT
        assert f(max_pos=4095) == tla.ERR_INVALID_ARGUMENT           # tables short of max_context_len 4096
        assert "cover" in tla.last_error()
        assert f(style=2) == tla.ERR_INVALID_ARGUMENT
    z = _kdesc(num_seqs=0)
    z.pre_rope_keys = 1
    assert L.tl_kivi_paged_attention_decode_pre_rope(ctypes.byref(z), *([FAKE] * 8), 0, FAKE, FAKE, 8192, 0, None,
                                                     0, None) == tla.OK


def test_kivi_rope_step_workspace_and_argument_checks():
    d = _kdesc(num_seqs=64)
    ws = tla.kivi_workspace_bytes(d, 4096)
    q_bytes, k_bytes = 64 * 32 * 128 * 2, 64 * 8 * 128 * 2
    a256 = lambda n: (n + 255) // 256 * 256
    assert tla.kivi_rope_step_workspace_bytes(d, 4096) == a256(ws) + a256(q_bytes) + k_bytes
    d16 = _kdesc(num_seqs=16)
    assert tla.kivi_rope_step_workspace_bytes(d16, 40000) == (
        a256(tla.kivi_workspace_bytes(d16, 40000)) + a256(16 * 32 * 128 * 2) + 16 * 8 * 128 * 2)
    assert tla.kivi_rope_step_workspace_bytes(_kdesc(head_size=64), 4096) == 0
    L = tla.lib
    need = tla.kivi_rope_step_workspace_bytes(d, 4096)

    def call(desc, max_pos=8192, style=0, ws_bytes=need, ws=FAKE, pos=FAKE):
        return L.tl_kivi_rope_decode_step(ctypes.byref(desc), FAKE, FAKE, FAKE, FAKE, pos, FAKE, FAKE, max_pos,
                                          style, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4096, ws, ws_bytes, None)
    assert call(d, ws_bytes=need - 1) == tla.ERR_INVALID_ARGUMENT
    assert "workspace" in tla.last_error()
    assert call(d, ws=None) == tla.ERR_INVALID_ARGUMENT
    assert call(d, max_pos=0) == tla.ERR_INVALID_ARGUMENT
    assert call(d, style=2) == tla.ERR_INVALID_ARGUMENT
    assert call(d, pos=None) == tla.ERR_INVALID_ARGUMENT
    assert call(_kdesc(head_size=64)) == tla.ERR_NOT_IMPLEMENTED
    assert call(_kdesc(num_seqs=0), ws=None, ws_bytes=0) == tla.OK


# ---- reference-named C++ operators (include/tl_truellm_ops.h) -------------

def _demangled_exports():
    import subprocess
    out = subprocess.run(["nm", "-DC", "--defined-only", tla.LIB_PATH], check=True, capture_output=True,
                         text=True).stdout
    return {ln.split(" ", 2)[2] for ln in out.splitlines() if len(ln.split(" ", 2)) == 3}


def test_exports_reference_named_operators():
    exp = _demangled_exports()
    want = [
        "reshape_and_cache(truellm::TrueBuffer const&, truellm::TrueBuffer const&, truellm::TrueBuffer&, "
        "truellm::TrueBuffer const&, ihipStream_t*)",
        "paged_attention_v1(truellm::TrueBuffer&, truellm::TrueBuffer const&, truellm::TrueBuffer const&, "
        "truellm::TrueBuffer const&, truellm::TrueBuffer const&, truellm::TrueBuffer const&, int, float, int, "
        "int, ihipStream_t*)",
        "paged_attention_v2(truellm::TrueBuffer&, truellm::TrueBuffer&, truellm::TrueBuffer&, "
        "truellm::TrueBuffer&, truellm::TrueBuffer const&, truellm::TrueBuffer const&, truellm::TrueBuffer "
        "const&, truellm::TrueBuffer const&, truellm::TrueBuffer const&, int, float, int, int, int, "
        "ihipStream_t*)",
        "truellm::kivi_params_supported(int, int, int)",
        "truellm::kivi_compress(__half const*, unsigned char*, int, int, int, int, ihipStream_t*)",
        "truellm::kivi_decompress(unsigned char const*, __half*, int, int, int, int, ihipStream_t*)",
        "copy_blocks(truellm::TrueBuffer&, truellm::TrueBuffer const&, ihipStream_t*)",
        "swap_blocks(truellm::TrueBuffer&, truellm::TrueBuffer&, truellm::TrueBuffer const&, int, ihipStream_t*)",
        "convert_fp8(truellm::TrueBuffer&, truellm::TrueBuffer const&, float, ihipStream_t*)",
        "truellm::vq_encode(__half const*, __half const*, unsigned short*, int, int, int, int, ihipStream_t*)",
        "truellm::vq_decode(__half*, __half const*, unsigned short const*, int, int, int, ihipStream_t*)",
        "truellm::codebook_init_kmeans(void const*, void*, int, int, int, int, ihipStream_t*)",
        "rms_norm(truellm::TrueBuffer&, truellm::TrueBuffer const&, truellm::TrueBuffer const&, float, ihipStream_t*)",
        "fused_add_rms_norm(truellm::TrueBuffer&, truellm::TrueBuffer&, truellm::TrueBuffer const&, "
        "truellm::TrueBuffer const&, float, ihipStream_t*)",
        "layer_norm(truellm::TrueBuffer&, truellm::TrueBuffer const&, truellm::TrueBuffer const&, "
        "truellm::TrueBuffer const&, float, ihipStream_t*)",
        "silu_and_mul(truellm::TrueBuffer&, truellm::TrueBuffer const&, truellm::TrueBuffer const&, ihipStream_t*)",
        "gelu_and_mul(truellm::TrueBuffer&, truellm::TrueBuffer const&, truellm::TrueBuffer const&, ihipStream_t*)",
        "gelu_tanh_and_mul(truellm::TrueBuffer&, truellm::TrueBuffer const&, truellm::TrueBuffer const&, "
        "ihipStream_t*)",
        "truellm_kernel_init",
    ]
    missing = [w for w in want if w not in exp]
    assert not missing, missing


class _Manifest(ctypes.Structure):
    _fields_ = [("abi_version", ctypes.c_uint32), ("name", ctypes.c_char_p), ("version", ctypes.c_char_p),
                ("category", ctypes.c_int), ("min_sm_major", ctypes.c_uint32), ("min_sm_minor", ctypes.c_uint32),
                ("initialize", ctypes.c_void_p), ("shutdown", ctypes.c_void_p), ("kernel_state", ctypes.c_void_p)]


def test_kernel_manifest():
    """kernel.h:23-57: ABI version 1, category ATTENTION, both hooks set."""
    fn = tla.lib.truellm_kernel_init
    fn.restype = ctypes.POINTER(_Manifest)
    m = fn().contents
    assert m.abi_version == 1 and m.category == 0
    assert m.name == b"tlattn_paged_attention_gfx950" and m.version
    assert (m.min_sm_major, m.min_sm_minor) == (9, 5)
    assert m.initialize and m.shutdown


def test_kivi_params_supported_shim_matches_reference_rule():
    f = tla.lib["_ZN7truellm21kivi_params_supportedEiii"]
    f.restype = ctypes.c_bool
    f.argtypes = [ctypes.c_int] * 3
    for args, want in [((128, 8, 16), True), ((129, 0, 16), False), ((64, 65, 16), False), ((64, 0, 0), False),
                       ((64, 64, 16), True), ((0, 0, 16), False), ((16, 17, 16), False), ((128, 8, 15), True)]:
        assert f(*args) == want, args


# ---- host-side callers: engine dispatch, allocator tables, compression pass --

def test_attention_plan_matches_engine_dispatch():
    """cuda_engine.cpp:1138-1160: v1 up to 32 blocks of context, else v2 with
    ceil(ctx / (32 bs)) partitions; scale 1/sqrt(d)."""
    assert tla.attention_plan(512, 16, 128)[:2] == (False, 1)
    assert tla.attention_plan(527, 16, 128)[:2] == (False, 1)       # 527 // 16 == 32
    assert tla.attention_plan(528, 16, 128)[:2] == (True, 2)
    assert tla.attention_plan(4096, 16, 128)[:2] == (True, 8)
    assert tla.attention_plan(32768, 16, 128)[:2] == (True, 64)
    assert tla.attention_plan(1055, 32, 128)[:2] == (False, 1)      # 1055 // 32 == 32
    assert tla.attention_plan(1056, 32, 128)[:2] == (True, 2)
    assert abs(tla.attention_plan(10, 16, 128)[2] - 1 / 128 ** 0.5) < 1e-7
    with pytest.raises(tla.TLError):
        tla.attention_plan(10, 0, 128)


def test_allocator_tables_and_slots():
    import numpy as np
    assert tla.max_blocks_per_seq(512) == 512 and tla.max_blocks_per_seq(100000) == 2048
    t = tla.build_block_tables([[7, 3, 9], [], [1]], 5)
    assert t.tolist() == [[7, 3, 9, -1, -1], [-1] * 5, [1, -1, -1, -1, -1]]
    with pytest.raises(tla.TLError):
        tla.build_block_tables([[1, 2, 3]], 2)
    blocks = np.array([5, 2, 11], np.int32)
    s = tla.build_slot_mapping(blocks, 16, 14, 5)
    assert s.tolist() == [5 * 16 + 14, 5 * 16 + 15, 2 * 16, 2 * 16 + 1, 2 * 16 + 2]
    # the decode step's single token at position L - 1
    assert tla.build_slot_mapping(blocks, 16, 47, 1).tolist() == [11 * 16 + 15]
    with pytest.raises(tla.TLError):
        tla.build_slot_mapping(blocks, 16, 47, 2)                      # needs a 4th block


def test_kivi_compression_pass_settings():
    """kv_compression_pass.cpp:29-66 (test_kv_compression_pass.cpp:40-108):
    residual_length -> n_outliers, bits 4 -> group 16 else 8, disabled when
    the parameters are unsupported; run_kivi skips empty layers and layers
    whose records exceed the scratch."""
    assert tla.kivi_pass_params(8, 4, 128) == (8, 16, True)
    assert tla.kivi_pass_params(8, 2, 128) == (8, 8, True)
    assert tla.kivi_pass_params(128, 4, 128) == (128, 16, False)       # > 64 outliers
    assert tla.kivi_pass_params(0, 4, 256) == (0, 16, False)           # head_dim > 128
    rec = tla.kivi_compressed_bytes(128, 8, 16)
    assert tla.kivi_pass_runs(10, 8, 128, 8, 16, 10 * 8 * rec)
    assert not tla.kivi_pass_runs(11, 8, 128, 8, 16, 10 * 8 * rec)
    assert not tla.kivi_pass_runs(0, 8, 128, 8, 16, 1 << 30)
