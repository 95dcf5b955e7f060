"""The golden cases: seeded inputs of the five workloads (reduced where the
full size would not fit a small fixture) and of the codecs.

tests/golden/make_golden.py runs the oracle on these inputs and writes
tests/golden/*.npz: for attention, the seed's input digest (SHA-256 of the
regenerated q / pools / tables / lengths) and the expected output in fp32;
for the codecs, the bytes themselves.  tests/test_golden.py checks the
oracle against the files (CPU) and the HIP kernels against them (GPU)."""
from __future__ import annotations

import hashlib
import math
import os

import numpy as np

import inputs
import oracle_lib as orc

GOLDEN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def load(name):
    return np.load(os.path.join(GOLDEN_DIR, name + ".npz"), allow_pickle=False)


# ---- attention workloads ---------------------------------------------------

def c1_fp16_batch4():
    """The CPU-path workload at full size: batch 4, 32 q / 8 kv heads, d 128,
    bs 16, lengths uniform in [128, 1024], a 512-block pool, fp16."""
    lens = inputs.uniform_lens(inputs.SEEDS[0], 4, 128, 1024)
    return inputs.make_paged_case(inputs.SEEDS[0], 4, 32, 8, 128, 16, lens, orc.F16, num_blocks=512, max_blocks=64)


def c2_bf16_varlen():
    """Llama-3-8B-shape decode, reduced to 8 sequences: lengths uniform in
    [512, 8192], bf16, a shuffled pool of 1.25x the blocks."""
    lens = inputs.uniform_lens(inputs.SEEDS[1], 8, 512, 8192)
    return inputs.make_paged_case(inputs.SEEDS[1], 8, 32, 8, 128, 16, lens, orc.BF16)


class KiviInputs:
    """KIVI INT4 workload reduced to 4 sequences: fp16 pools with 4 outlier K
    channels per kv head scaled x8, a shuffled page table, R = 128."""

    def __init__(self):
        seed = inputs.SEEDS[2]
        self.lens = np.array([4096, 4100, 3000, 200], np.int32)
        self.R = 128
        base = inputs.make_paged_case(seed, 4, 32, 8, 128, 16, self.lens, orc.F32)
        rng = np.random.default_rng(seed + 1)
        for h in range(8):
            ch = rng.choice(128, size=4, replace=False)
            base.k_cache[:, h, ch, :] *= 8
        self.k = inputs.encode(base.k_cache, orc.F16)
        self.v = inputs.encode(base.v_cache, orc.F16)
        self.q = inputs.encode(orc.bits_to_f32(base.q, orc.F32), orc.F16)
        self.tables, self.scale = base.tables, base.scale
        max_pages = int(self.lens.max()) // 32 + 1
        self.num_pages = 4 * max_pages + 3
        self.page_tables = rng.permutation(self.num_pages)[: 4 * max_pages].astype(np.int32).reshape(4, max_pages)

    def pages(self):
        pages = np.zeros((self.num_pages, 8, orc.KIVI_PAGE_BYTES), np.uint8)
        orc.kivi_build_pages(self.k, self.v, self.tables, self.lens, self.R, pages, self.page_tables)
        return pages

    def digest(self):
        return digest(self.q, self.k, self.v, self.tables, self.lens, self.page_tables)


class Fp8Inputs:
    """FP8 E4M3 long-context workload reduced to 2 sequences of 8192 tokens:
    per-tensor scales absmax / 448 over N(0, 1) pools, bf16 q."""

    def __init__(self):
        base = inputs.make_paged_case(inputs.SEEDS[3], 2, 32, 8, 128, 16, [8192, 8192], orc.F32)
        self.ks = float(np.abs(base.k_cache).max()) / 448.0
        self.vs = float(np.abs(base.v_cache).max()) / 448.0
        self.k8 = orc.f32_to_e4m3(base.k_cache, np.float32(1.0) / np.float32(self.ks))
        self.v8 = orc.f32_to_e4m3(base.v_cache, np.float32(1.0) / np.float32(self.vs))
        self.q = inputs.encode(orc.bits_to_f32(base.q, orc.F32), orc.BF16)
        self.tables, self.lens, self.scale = base.tables, base.seq_lens, base.scale

    def digest(self):
        return digest(self.q, self.k8, self.v8, self.tables, self.lens)


class PrefillInputs:
    """Chunked prefill reduced to 16 q / 2 kv heads: a 512-token chunk with a
    512-token prefix, a first 512-token chunk and 4 decode rows at 1024, bf16."""

    def __init__(self):
        shape = [(512, 1024), (512, 512), (1, 1024), (1, 1024), (1, 700), (1, 1)]
        self.q_lens = np.array([a for a, _ in shape], np.int32)
        self.lens = np.array([b for _, b in shape], np.int32)
        seed = inputs.SEEDS[4]
        self.case = inputs.make_paged_case(seed, len(shape), 16, 2, 128, 16, self.lens, orc.BF16)
        self.cu = np.concatenate([[0], np.cumsum(self.q_lens)]).astype(np.int32)
        rng = np.random.default_rng(seed + 7)
        self.q = inputs.encode(rng.standard_normal((int(self.cu[-1]), 16, 128), dtype=np.float32), orc.BF16)
        # the rows kept in the fixture: every 32nd row of each chunk, its
        # last row, and every decode row
        self.rows = np.unique(np.concatenate([np.arange(0, 512, 32), [511], 512 + np.arange(0, 512, 32), [1023],
                                              np.arange(1024, int(self.cu[-1]))])).astype(np.int64)

    def digest(self):
        c = self.case
        return digest(self.q, c.k_cache, c.v_cache, c.tables, self.lens, self.cu)


# ---- codecs ----------------------------------------------------------------

def kivi_vectors(D, n=64):
    """n fp16 vectors of D channels: N(0, 1) times 4, a constant vector,
    one with large outliers and one of tiny values."""
    rng = np.random.default_rng(inputs.SEEDS[2] + D)
    x = (rng.standard_normal((n, D)) * 4).astype(np.float32)
    x[0] = 2.5
    x[1, ::7] *= 100
    x[2] *= 1e-4
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def kivi_page_tokens():
    rng = np.random.default_rng(inputs.SEEDS[2] + 99)
    k = rng.standard_normal((32, 128)).astype(np.float32)
    k[:, [5, 77]] *= 8
    v = rng.standard_normal((32, 128)).astype(np.float32)
    f16 = lambda a: a.astype(np.float16).view(np.uint16).reshape(32, 128)
    return f16(k), f16(v)


KIVI_VEC_PARAMS = [(128, 8, 16), (64, 4, 16)]
ATTENTION_SCALE = 1 / math.sqrt(128)


# ---- KIVI vector codec: known answers derived by hand ---------------------

# Records whose outliers the reference writes in selection-slot order
# (kivi_cache.cu:50-60 replaces the first minimum of the slot array, strict
# '>' on |x|; :73-78 write the slots in array order), derived by hand.
KIVI_SLOT_ORDER_CASES = [
    # x = [1, 5, 7, 0.5], O = 2, G = 2.  Scan: d0 -> slot 0 (min now slot 1
    # at -1); d1 -> slot 1 (min slot 0 = 1); d2 (7 > 1) replaces slot 0;
    # d3 (0.5 < 5) stays out.  Slots: (2, 7), (1, 5): neither channel order
    # (1, 2) nor magnitude order (2, 1) read the other way.  Residual
    # channels 0, 3 = [1, 0.5]: gmin 0.5, range 0.5, scale 30 -> codes 15, 0
    # (byte 0x0F); step fp16(1/30) = 0x2844, zero fp16(0.5) = 0x3800.
    ([1.0, 5.0, 7.0, 0.5], 2, 2,
     [0x02, 0x00, 0x47, 0x01, 0x00, 0x45, 0x0F, 0x44, 0x28, 0x00, 0x38]),
    # x = [3, 1, 4, 1.5, -5, 3], O = 3, G = 2.  Scan: d0 slot 0, d1 slot 1,
    # d2 slot 2 (min slot 1 = 1); d3 (1.5 > 1) replaces slot 1 mid-scan
    # (min slot 1 = 1.5); d4 (|-5| > 1.5) replaces slot 1 again (min slot 0
    # = 3); d5 (3, a tie with the minimum) stays out.  Slots: (0, 3), (4, -5),
    # (2, 4): channel order would be 0, 2, 4 and magnitude order 4, 2, 0.
    # Residual channels 1, 3, 5 = [1, 1.5, 3]: group [1, 1.5] -> scale 30,
    # codes 0, 15 (0xF0), step 0x2844, zero fp16(1) = 0x3C00; group [3]
    # (one channel, degenerate) -> code 0, step 0, zero fp16(3) = 0x4200.
    ([3.0, 1.0, 4.0, 1.5, -5.0, 3.0], 3, 2,
     [0x00, 0x00, 0x42, 0x04, 0x00, 0xC5, 0x02, 0x00, 0x44,
      0xF0, 0x44, 0x28, 0x00, 0x3C, 0x00, 0x00, 0x00, 0x00, 0x42]),
]
