"""tl_paged_attention_decode_noalloc: the decode with the library's own
split-K scratch, against tl_paged_attention_decode with a caller workspace.

Both run the same kernels on the same plan, so the outputs must be equal
bit for bit (a stronger bar than the 2e-3 of the decode parity tests); the
smaller call is also checked against the oracle.  Two calls in a row, the
second smaller, show that the scratch's leftover contents from the first
call do not leak into the second."""
import ctypes
import math

import numpy as np
import pytest
import torch

import inputs
import oracle_lib as orc
import tl_attn as tla

FAKE = ctypes.c_void_p(0x1000)  # never dereferenced: the call fails on the host


def _desc(S, H, n_kv, pt, kv_dtype=tla.BF16, q_dtype=tla.BF16):
    d = tla.DecodeDesc()
    d.num_seqs, d.num_heads, d.num_kv_heads, d.head_size, d.block_size = S, H, n_kv, 128, 16
    d.max_blocks_per_seq, d.num_blocks = 4096, 1 << 20
    d.q_dtype, d.kv_dtype, d.gqa_map, d.partition_tokens = q_dtype, kv_dtype, tla.GQA_GROUPED, pt
    d.scale, d.k_scale, d.v_scale = 1 / math.sqrt(128), 1.0, 1.0
    return d


def test_noalloc_rejects_a_plan_beyond_the_scratch():
    """64 sequences of 32768 tokens, 32 q heads, 512-token partitions: 64
    partitions need 68 MB of partials, more than the 32 MiB scratch (the
    16-sequence case of the same shape needs 17 MB and fits).  The check
    runs on the host before any HIP call."""
    assert tla.workspace_bytes(_desc(16, 32, 8, 512, kv_dtype=tla.FP8_E4M3), 32768) == 16 * 32 * 64 * 520
    d = _desc(64, 32, 8, 512, kv_dtype=tla.FP8_E4M3)
    need = tla.workspace_bytes(d, 32768)
    assert need == 64 * 32 * 64 * (128 + 2) * 4 > tla.NOALLOC_SCRATCH_BYTES
    rc = tla.lib.tl_paged_attention_decode_noalloc(ctypes.byref(d), FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                                                   32768, None)
    assert rc == tla.ERR_INVALID_ARGUMENT
    assert b"scratch" in tla.lib.tl_last_error_string()
    # argument errors come from the decode's own checks
    d.num_heads = 30
    rc = tla.lib.tl_paged_attention_decode_noalloc(ctypes.byref(d), FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                                                   100, None)
    assert rc == tla.ERR_INVALID_ARGUMENT


def _run_pair(case, pt, code, kv_dtype=None, k_scale=1.0, v_scale=1.0, kv=None):
    """The same decode through both entry points; returns (noalloc, caller-workspace) outputs."""
    from gpu_util import dev
    q = dev(case.q, code)
    k = dev(case.k_cache, code) if kv is None else kv[0]
    v = dev(case.v_cache, code) if kv is None else kv[1]
    bt, sl = dev(case.tables), dev(case.seq_lens)
    desc = tla.make_decode_desc(q, k, bt, case.num_kv_heads, case.scale, kv_dtype=kv_dtype,
                                gqa_map=tla.GQA_GROUPED, partition_tokens=pt, k_scale=k_scale,
                                v_scale=v_scale)
    max_ctx = int(case.seq_lens.max())
    need = tla.workspace_bytes(desc, max_ctx)
    assert 0 < need <= tla.NOALLOC_SCRATCH_BYTES, need
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    a = torch.full_like(q, float("nan"))
    b = torch.full_like(q, float("nan"))
    tla.paged_attention_decode_noalloc(desc, a, q, k, v, bt, sl, max_ctx)
    tla.paged_attention_decode(desc, b, q, k, v, bt, sl, max_ctx, ws)
    torch.cuda.synchronize()
    return a, b


@pytest.mark.gpu
def test_noalloc_matches_caller_workspace_twice_second_smaller():
    from gpu_util import assert_close
    # 1) batch 64, ctx 4096, 32/8 heads, bf16, 512-token partitions (8.5 MB of partials)
    big = inputs.make_paged_case(inputs.SEEDS[1], 64, 32, 8, 128, 16, [4096] * 64, orc.BF16)
    print("case noalloc call 1: bf16 B=64 ctx 4096 split-K 512", flush=True)
    a, b = _run_pair(big, 512, orc.BF16)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    # 2) smaller: batch 6, mixed lengths with holes, f16, 1024-token partitions
    lens = [3000, 1, 700, 1025, 2048, 5]
    small = inputs.make_paged_case(77, 6, 32, 8, 128, 16, lens, orc.F16, holes=3)
    print("case noalloc call 2: f16 B=6 mixed lengths split-K 1024", flush=True)
    a, b = _run_pair(small, 1024, orc.F16)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    ref = orc.paged_attention(small.q, orc.F16, small.k_cache, small.v_cache, orc.F16, small.tables,
                              small.seq_lens, 8, small.scale, orc.GROUPED)
    assert_close(a, ref, orc.F16, 2e-3, "noalloc small")


@pytest.mark.gpu
def test_noalloc_fp8_and_single_pass():
    """FP8 KV at 512-token partitions (batch 4, ctx 8192), then a plan that
    runs single pass (no scratch used)."""
    from gpu_util import dev
    case = inputs.make_paged_case(inputs.SEEDS[3], 4, 32, 8, 128, 16, [8192, 8000, 4097, 512], orc.F32)
    ks = float(np.abs(case.k_cache).max()) / 448
    vs = float(np.abs(case.v_cache).max()) / 448
    k8 = dev(orc.f32_to_e4m3(case.k_cache, 1 / ks))
    v8 = dev(orc.f32_to_e4m3(case.v_cache, 1 / vs))
    case.q = inputs.encode(case.q, orc.BF16)
    print("case noalloc fp8 B=4 ctx 8192 split-K 512", flush=True)
    a, b = _run_pair(case, 512, orc.BF16, kv_dtype=tla.FP8_E4M3, k_scale=ks, v_scale=vs, kv=(k8, v8))
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    small = inputs.make_paged_case(78, 3, 32, 8, 128, 16, [100, 33, 16], orc.BF16)
    q, k, v = dev(small.q, orc.BF16), dev(small.k_cache, orc.BF16), dev(small.v_cache, orc.BF16)
    bt, sl = dev(small.tables), dev(small.seq_lens)
    desc = tla.make_decode_desc(q, k, bt, 8, small.scale, partition_tokens=-1)
    assert tla.workspace_bytes(desc, 100) == 0
    a = torch.full_like(q, float("nan"))
    b = torch.full_like(q, float("nan"))
    print("case noalloc single pass", flush=True)
    tla.paged_attention_decode_noalloc(desc, a, q, k, v, bt, sl, 100)
    tla.paged_attention_decode(desc, b, q, k, v, bt, sl, 100)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


# A fresh process whose first call of the library on the GPU is
# tl_paged_attention_decode_noalloc inside a stream capture: the scratch
# address lookup happens there.  The graph is replayed three times with eager
# work between, each replay checked bit for bit against the caller-workspace
# entry point run eagerly after the capture.
_FIRST_CALL_IN_CAPTURE = r"""
import sys
sys.path[:0] = sys.argv[1:3]
import torch
import inputs
import oracle_lib as orc
import tl_attn as tla
from gpu_util import dev

torch.cuda.set_device(0)
case = inputs.make_paged_case(79, 8, 32, 8, 128, 16, [4096, 3000, 1, 700, 1025, 2048, 5, 4000], orc.BF16,
                              holes=2)
q, k, v = dev(case.q, orc.BF16), dev(case.k_cache, orc.BF16), dev(case.v_cache, orc.BF16)
bt, sl = dev(case.tables), dev(case.seq_lens)
max_ctx = int(case.seq_lens.max())
desc = tla.make_decode_desc(q, k, bt, 8, case.scale, gqa_map=tla.GQA_GROUPED, partition_tokens=512)
assert tla.workspace_bytes(desc, max_ctx) > 0
out = torch.zeros_like(q)
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
cap = torch.cuda.Stream()
print("case noalloc first call inside a stream capture", flush=True)
with torch.cuda.graph(graph, stream=cap):
    tla.paged_attention_decode_noalloc(desc, out, q, k, v, bt, sl, max_ctx, cap)
ws = torch.empty(tla.workspace_bytes(desc, max_ctx), dtype=torch.uint8, device="cuda")
want = torch.full_like(q, float("nan"))
tla.paged_attention_decode(desc, want, q, k, v, bt, sl, max_ctx, ws)
torch.cuda.synchronize()
for i in range(3):
    out.zero_()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), want.view(torch.int16)), f"replay {i}"
    tla.paged_attention_decode_noalloc(desc, out, q, k, v, bt, sl, max_ctx)   # eager, between replays
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), want.view(torch.int16)), f"eager {i}"
print("first-call capture ok", flush=True)
"""


@pytest.mark.gpu
def test_noalloc_first_call_inside_stream_capture():
    import os
    import subprocess
    import sys
    here = os.path.dirname(os.path.abspath(__file__))
    pkg = os.path.join(os.path.dirname(here), "truellm-engine_amd")
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_IN_CAPTURE, here, pkg], capture_output=True,
                       text=True, timeout=300)
    print(r.stdout[-2000:], r.stderr[-4000:], flush=True)
    assert r.returncode == 0 and "first-call capture ok" in r.stdout
