"""Seeded synthetic inputs for the paged-attention workloads.

Shapes follow the engine's data contract: q [S, H, D]; pools
[N, n_kv, D, BS]; block tables int32 [S, max_blocks] padded with -1
(cuda_allocator.cpp:231-253); physical blocks drawn from a shuffled pool.
Element data are numpy bit patterns (uint16 for f16/bf16, float32 for f32)
so the oracle and the GPU see identical bytes.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

import oracle_lib as orc

# seeds of the five workloads (paged-attention decode fp16 at batch 4, bf16 at
# batch 64, KIVI INT4, FP8 long context, chunked prefill)
SEEDS = [0x7E5E0001, 0x7E5E0002, 0x7E5E0003, 0x7E5E0004, 0x7E5E0005]


@dataclass
class PagedCase:
    q: np.ndarray          # [S, H, D] bits / f32
    k_cache: np.ndarray    # [N, n_kv, D, BS]
    v_cache: np.ndarray
    tables: np.ndarray     # int32 [S, max_blocks]
    seq_lens: np.ndarray   # int32 [S]
    code: int              # oracle dtype code of q and the pools
    num_kv_heads: int
    scale: float

    @property
    def shape(self):
        S, H, D = self.q.shape
        return S, H, D, self.k_cache.shape[3]


def encode(x: np.ndarray, code: int) -> np.ndarray:
    if code == orc.F16:
        return orc.f32_to_f16_bits(x)
    if code == orc.BF16:
        return orc.f32_to_bf16_bits(x)
    if code == orc.F32:
        return np.ascontiguousarray(x, np.float32)
    raise ValueError(code)


def make_paged_case(seed, S, H, n_kv, D, BS, lens, code, num_blocks=None, pool_factor=1.25,
                    max_blocks=None, holes=0) -> PagedCase:
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, np.int32)
    nblk = [(int(L) + BS - 1) // BS for L in lens]
    total = sum(nblk)
    N = num_blocks if num_blocks is not None else max(1, math.ceil(pool_factor * total))
    assert N >= total, "pool too small"
    mb = max_blocks if max_blocks is not None else max(1, max(nblk) if nblk else 1)
    perm = rng.permutation(N).astype(np.int32)
    tables = np.full((S, mb), -1, np.int32)
    off = 0
    for s in range(S):
        tables[s, :nblk[s]] = perm[off:off + nblk[s]]
        off += nblk[s]
    for _ in range(holes):                      # punch table holes inside sequences
        s = int(rng.integers(S))
        if nblk[s] > 1:
            tables[s, int(rng.integers(nblk[s]))] = -1
    q = encode(rng.standard_normal((S, H, D), dtype=np.float32), code)
    k = encode(rng.standard_normal((N, n_kv, D, BS), dtype=np.float32), code)
    v = encode(rng.standard_normal((N, n_kv, D, BS), dtype=np.float32), code)
    return PagedCase(q, k, v, tables, lens, code, n_kv, 1.0 / math.sqrt(D))


def uniform_lens(seed, S, lo, hi):
    rng = np.random.default_rng(seed ^ 0x5EED)
    return rng.integers(lo, hi + 1, size=S).astype(np.int32)
