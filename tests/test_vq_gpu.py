"""VQ codec on the GPU: encode / decode / k-means bit-exact against the
oracle, the reference's own test cases, the reference-named operators, and
graph replay."""
import ctypes

import numpy as np
import pytest
import torch

import oracle_lib as orc
import tl_attn as tla
from gpu_util import dev, host_bits

pytestmark = pytest.mark.gpu


def _f16(x):
    return orc.f32_to_f16_bits(np.asarray(x, np.float32))


def _idx_dev(n):
    return torch.zeros(n, dtype=torch.int16, device="cuda")


def _encode_dev(kv_bits, book_bits):
    kv, book = dev(kv_bits, orc.F16), dev(book_bits, orc.F16)
    idx = _idx_dev(kv_bits.size // book_bits.shape[1])
    tla.vq_encode(kv, book, idx)
    torch.cuda.synchronize()
    return idx.cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("n,K,D", [(512, 256, 128), (37, 1000, 64), (1000, 17, 8), (5, 300, 256),
                                   (4099, 256, 128)])
def test_vq_encode_bit_exact(n, K, D):
    rng = np.random.default_rng(n + K + D)
    book = _f16(rng.standard_normal((K, D)))
    kv = _f16(rng.standard_normal((n, D)))
    kv[::11] = book[rng.integers(0, K, size=len(kv[::11]))]   # exact copies
    if K > 3:
        book[K - 1] = book[1]                                  # duplicate entry
    kv[2] = book[1]
    kv[min(3, n - 1), 0] = 0x7E00                              # NaN
    print(f"case vq encode n={n} K={K} D={D}", flush=True)
    assert np.array_equal(_encode_dev(kv, book), orc.vq_encode(kv, book))


def test_vq_reference_known_answers_on_gpu():
    """test_vq_kernels.cpp:96-204 through the library."""
    book = _f16([[c * 10 + d for d in range(8)] for c in range(4)])
    want = np.array([(t * 2 + h) % 4 for t in range(4) for h in range(2)], np.uint16)
    assert np.array_equal(_encode_dev(book[want], book), want)
    book2 = _f16([[0] * 4, [1000] * 4, [2000] * 4])
    kv2 = _f16([[0.5, -0.5, 0.2, -0.2], [1001, 999, 1000.5, 999.5], [1999, 2001, 1999.5, 2000.5]])
    # head_dim 4 is below the library's 8-element rows: pad both with zeros (distances unchanged)
    pad = lambda a: np.concatenate([a, np.zeros((a.shape[0], 4), np.uint16)], 1)
    assert np.array_equal(_encode_dev(pad(kv2), pad(book2)), np.array([0, 1, 2], np.uint16))


def test_vq_decode_bit_exact_and_out_of_range_rows():
    rng = np.random.default_rng(60)
    K, D, n = 300, 128, 777
    book = _f16(rng.standard_normal((K, D)))
    idx = rng.integers(0, K, size=n).astype(np.uint16)
    idx[::13] = K + 5                                          # out of range: row untouched
    out0 = _f16(rng.standard_normal((n, D)))
    outd = dev(out0, orc.F16)
    print("case vq decode", flush=True)
    tla.vq_decode(outd, dev(book, orc.F16), torch.from_numpy(idx.view(np.int16)).cuda())
    torch.cuda.synchronize()
    ref = out0.copy()
    orc.vq_decode(ref, book, idx)
    assert np.array_equal(host_bits(outd), ref)


def test_vq_kmeans_bit_exact_and_deterministic():
    """4096 samples, 256 entries, d 128, seeded with the first 256 samples
    (Forgy), 3 iterations: the book equals the oracle's bit for bit, and a
    second run gives the same bytes."""
    rng = np.random.default_rng(61)
    n, K, D, iters = 4096, 256, 128, 3
    centres = rng.standard_normal((32, D)) * 4
    data = _f16(centres[rng.integers(0, 32, size=n)] + rng.standard_normal((n, D)))
    book0 = data[:K].copy()
    ws = torch.empty(tla.vq_kmeans_workspace_bytes(n, K, D), dtype=torch.uint8, device="cuda")
    dd = dev(data, orc.F16)
    runs = []
    for _ in range(2):
        bd = dev(book0, orc.F16)
        print("case vq kmeans", flush=True)
        tla.vq_kmeans(dd, bd, iters, ws)
        torch.cuda.synchronize()
        runs.append(host_bits(bd))
    ref = book0.copy()
    orc.vq_kmeans(data, ref, iters)
    assert np.array_equal(runs[0], ref)
    assert np.array_equal(runs[1], ref)


def test_vq_encode_graph_replay():
    rng = np.random.default_rng(62)
    K, D, n = 256, 128, 512
    book, kv = dev(_f16(rng.standard_normal((K, D))), orc.F16), dev(_f16(rng.standard_normal((n, D))), orc.F16)
    idx = _idx_dev(n)
    tla.vq_encode(kv, book, idx)
    torch.cuda.synchronize()
    eager = idx.clone()
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=cap):
        tla.vq_encode(kv, book, idx, cap)
    for _ in range(3):
        idx.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(idx, eager)


def _fn(mangled, argtypes):
    f = tla.lib[mangled]
    f.argtypes = argtypes
    f.restype = None
    return f


def test_vq_shims_equal_c_abi():
    enc = _fn("_ZN7truellm9vq_encodeEPK6__halfS2_PtiiiiP12ihipStream_t",
              [ctypes.c_void_p] * 3 + [ctypes.c_int] * 4 + [ctypes.c_void_p])
    dec = _fn("_ZN7truellm9vq_decodeEP6__halfPKS0_PKtiiiP12ihipStream_t",
              [ctypes.c_void_p] * 3 + [ctypes.c_int] * 3 + [ctypes.c_void_p])
    km = _fn("_ZN7truellm20codebook_init_kmeansEPKvPviiiiP12ihipStream_t",
             [ctypes.c_void_p] * 2 + [ctypes.c_int] * 4 + [ctypes.c_void_p])
    rng = np.random.default_rng(63)
    S, n_kv, D, K = 64, 8, 128, 256
    kv_bits = _f16(rng.standard_normal((S, n_kv, D)))
    book_bits = _f16(rng.standard_normal((K, D)))
    kv, book = dev(kv_bits, orc.F16), dev(book_bits, orc.F16)
    a, b = _idx_dev(S * n_kv), _idx_dev(S * n_kv)
    st = torch.cuda.current_stream().cuda_stream
    print("case vq shims", flush=True)
    enc(kv.data_ptr(), book.data_ptr(), a.data_ptr(), S, n_kv, D, K, st)
    tla.vq_encode(kv, book, b)
    out = torch.zeros_like(kv)
    dec(out.data_ptr(), book.data_ptr(), a.data_ptr(), S, n_kv, D, st)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert np.array_equal(host_bits(out).reshape(-1, D), book_bits[a.cpu().numpy().view(np.uint16)])
    data = dev(_f16(rng.standard_normal((2048, D))), orc.F16)
    b1, b2 = book.clone(), book.clone()
    ws = torch.empty(tla.vq_kmeans_workspace_bytes(2048, K, D), dtype=torch.uint8, device="cuda")
    km(data.data_ptr(), b1.data_ptr(), 2048, K, D, 2, st)
    tla.vq_kmeans(data, b2, 2, ws)
    torch.cuda.synchronize()
    assert torch.equal(b1.view(torch.int16), b2.view(torch.int16))
