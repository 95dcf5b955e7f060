"""Block management on the GPU (copy_blocks, swap_blocks): bit-exact
against the oracle, the reference-named operators against the C ABI, and
graph replay."""
import ctypes

import numpy as np
import pytest
import torch

import oracle_lib as orc
import tl_attn as tla

pytestmark = pytest.mark.gpu


def _pool(rng, n, shape, dtype):
    """Random bytes viewed as dtype (NaN payloads and all)."""
    nbytes = int(np.prod(shape)) * torch.tensor([], dtype=dtype).element_size()
    raw = torch.from_numpy(rng.integers(0, 256, size=(n, nbytes), dtype=np.uint8))
    return raw.view(dtype).reshape((n,) + shape).contiguous()


def _bytes(t):
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


def _mapping(rng, N, P, bad=True):
    perm = rng.permutation(N)
    m = np.stack([perm[:P], perm[P:2 * P]], 1).astype(np.int32)
    if bad:
        m = np.concatenate([m, np.array([[-1, 0], [0, N], [N + 3, 1]], np.int32)])
    return m


@pytest.mark.parametrize("dtype,shape", [(torch.float16, (8, 128, 16)), (torch.bfloat16, (2, 64, 32)),
                                         (torch.float32, (4, 128, 16)), (torch.uint8, (8, 128, 16)),
                                         (torch.uint8, (3, 5, 7))])
def test_copy_blocks_bit_exact(dtype, shape):
    """Both pools, the 16-byte path and (3 x 5 x 7 bytes) the byte path;
    out-of-range pairs skipped."""
    rng = np.random.default_rng(31)
    N, P = 96, 40
    k, v = _pool(rng, N, shape, dtype), _pool(rng, N, shape, dtype)
    m = _mapping(rng, N, P)
    kd, vd, md = k.cuda(), v.cuda(), torch.from_numpy(m).cuda()
    print(f"case copy_blocks {dtype} {shape}", flush=True)
    tla.copy_blocks(kd, vd, md)
    torch.cuda.synchronize()
    kh, vh = _bytes(k).reshape(N, -1).copy(), _bytes(v).reshape(N, -1).copy()
    orc.copy_blocks(kh, vh, m)
    assert np.array_equal(_bytes(kd).reshape(N, -1), kh)
    assert np.array_equal(_bytes(vd).reshape(N, -1), vh)


def test_copy_blocks_full_size():
    """2048 pairs of 32 KiB blocks (fp16, 8 kv heads, d 128, bs 16) out of a
    4096-block pool: every destination equals its source, every other block
    is untouched (checked against torch indexing on the device)."""
    g = torch.Generator(device="cuda").manual_seed(32)
    N, P = 4096, 2048
    k = torch.randn(N, 8, 128, 16, generator=g, device="cuda", dtype=torch.float16)
    v = torch.randn(N, 8, 128, 16, generator=g, device="cuda", dtype=torch.float16)
    perm = torch.randperm(N, generator=g, device="cuda")
    src, dst = perm[:P], perm[P:]
    m = torch.stack([src, dst], 1).to(torch.int32).contiguous()
    ek, ev = k.clone(), v.clone()
    ek[dst] = k[src]
    ev[dst] = v[src]
    print("case copy_blocks full size", flush=True)
    tla.copy_blocks(k, v, m)
    torch.cuda.synchronize()
    assert torch.equal(k.view(torch.int16), ek.view(torch.int16))
    assert torch.equal(v.view(torch.int16), ev.view(torch.int16))


@pytest.mark.parametrize("shape", [(8, 128, 16), (3, 5, 7)])
def test_swap_blocks_round_trip_pinned_host(shape):
    """Out to a pinned host buffer and back, each direction bit-exact against
    the oracle; ids outside either pool skip the pair."""
    rng = np.random.default_rng(33)
    N, M = 64, 24
    pool = _pool(rng, N, shape, torch.float16).cuda()
    host = torch.zeros((M,) + shape, dtype=torch.float16, pin_memory=True)
    src = rng.permutation(N)[:16].astype(np.int32)
    slots = rng.permutation(M)[:16].astype(np.int32)
    out_map = np.concatenate([np.stack([src, slots], 1), [[N, 0], [0, M], [-2, 3]]]).astype(np.int32)
    print(f"case swap_blocks out {shape}", flush=True)
    ph, hh = _bytes(pool).reshape(N, -1).copy(), np.zeros((M, _bytes(pool).reshape(N, -1).shape[1]), np.uint8)
    tla.swap_blocks(pool, host, torch.from_numpy(out_map).cuda(), 0)
    torch.cuda.synchronize()
    orc.swap_blocks(ph, hh, out_map, 0)
    assert np.array_equal(host.view(torch.uint8).reshape(M, -1).numpy(), hh)
    saved = pool[torch.from_numpy(src).long().cuda()].clone()
    pool[torch.from_numpy(src).long().cuda()] = 0
    back = np.stack([slots, src], 1).astype(np.int32)
    print(f"case swap_blocks in {shape}", flush=True)
    tla.swap_blocks(pool, host, torch.from_numpy(back).cuda(), 1)
    torch.cuda.synchronize()
    assert torch.equal(pool[torch.from_numpy(src).long().cuda()].view(torch.int16), saved.view(torch.int16))


def test_copy_blocks_graph_replay():
    rng = np.random.default_rng(34)
    N = 64
    k0, v0 = _pool(rng, N, (8, 128, 16), torch.bfloat16).cuda(), _pool(rng, N, (8, 128, 16), torch.bfloat16).cuda()
    m = torch.from_numpy(_mapping(rng, N, 20, bad=False)).cuda()
    k, v = k0.clone(), v0.clone()
    print("case copy_blocks graph", flush=True)
    tla.copy_blocks(k, v, m)
    torch.cuda.synchronize()
    ek, ev = k.clone(), v.clone()
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=cap):
        tla.copy_blocks(k, v, m, cap)
    for _ in range(3):
        k.copy_(k0)
        v.copy_(v0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(k.view(torch.int16), ek.view(torch.int16))
        assert torch.equal(v.view(torch.int16), ev.view(torch.int16))
