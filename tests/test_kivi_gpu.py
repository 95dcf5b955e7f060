"""KIVI INT4 on the GPU against the oracle.

Codec bytes (records, pages, nibbles, scales, zeros) must be bit-exact;
decode attention is compared with attention on the oracle's dequantised
pages plus the fp16 residual window, max-abs 1e-2 (plus half an fp16 ulp)."""
import math

import numpy as np
import pytest
import torch

import golden_cases
import inputs
import oracle_lib as orc
import tl_attn as tla
from gpu_util import assert_close, dev, host_bits

pytestmark = pytest.mark.gpu

ATOL_KIVI = 1e-2


def _f16(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


# ---------------------------------------------------------------------------
# reference vector codec
# ---------------------------------------------------------------------------

def _special_vectors(rng, n, D):
    x = rng.standard_normal((n, D)).astype(np.float32)
    x[0] = 2.5                                   # degenerate groups
    x[1, : D // 2] = 0.0                         # constant halves
    x[2] = np.round(x[2] * 4) / 4                # many exact ties
    x[3, 5] = 60000.0                            # large outlier
    x[4] *= 1e-4                                 # tiny values
    x[5, 0::2] = -x[5, 1::2]                   # +-pairs of equal magnitude
    return x


@pytest.mark.parametrize("D,O,G", [(128, 8, 16), (64, 4, 16), (64, 0, 16), (32, 0, 16),
                                   (100, 3, 10), (128, 64, 16), (64, 64, 16), (128, 0, 32),
                                   (96, 13, 8)])
def test_vector_codec_bit_exact(D, O, G):
    rng = np.random.default_rng(D * 131 + O * 7 + G)
    n = 300
    xb = _f16(_special_vectors(rng, n, D)).reshape(n, D)
    stride = orc.kivi_compressed_bytes(D, O, G)
    want = np.full(n * stride, 0xAB, np.uint8)
    orc.kivi_compress(xb, D, O, G, out=want)
    rec = torch.full((n * stride,), 0xAB, dtype=torch.uint8, device="cuda")
    print(f"case vec codec D={D} O={O} G={G}", flush=True)
    tla.kivi_compress(dev(xb, orc.F16), rec, n, D, O, G)
    torch.cuda.synchronize()
    got = rec.cpu().numpy()
    assert np.array_equal(got, want)
    back = torch.zeros(n, D, dtype=torch.float16, device="cuda")
    tla.kivi_decompress(rec, back, n, D, O, G)
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(back).ravel(), orc.kivi_decompress(want, n, D, O, G))


def test_vector_codec_hand_derived_slot_order():
    """The kernel writes the outliers in the reference's selection-slot order
    (kivi_cache.cu:50-78), byte for byte against records derived by hand
    (not by the oracle): O = 2 and O = 3 with a mid-scan replacement, a
    negative outlier and a tie with the running minimum."""
    for x, O, G, want in golden_cases.KIVI_SLOT_ORDER_CASES:
        D = len(x)
        print(f"case vec codec hand-derived D={D} O={O} G={G}", flush=True)
        rec = torch.full((len(want),), 0xAB, dtype=torch.uint8, device="cuda")
        tla.kivi_compress(dev(_f16(x).reshape(1, D), orc.F16), rec, 1, D, O, G)
        back = torch.zeros(1, D, dtype=torch.float16, device="cuda")
        tla.kivi_decompress(rec, back, 1, D, O, G)
        torch.cuda.synchronize()
        assert [int(b) for b in rec.cpu().numpy()] == want
        assert back.float().cpu().numpy().ravel().tolist() == x


def test_vector_codec_reference_roundtrips():
    """test_kivi_roundtrip.cpp:83-200 on the GPU path."""
    def rt(x, D, O, G):
        n = x.size // D
        xd = dev(_f16(x).reshape(n, D), orc.F16)
        rec = torch.zeros(n * tla.kivi_compressed_bytes(D, O, G), dtype=torch.uint8, device="cuda")
        out = torch.zeros(n, D, dtype=torch.float16, device="cuda")
        tla.kivi_compress(xd, rec, n, D, O, G)
        tla.kivi_decompress(rec, out, n, D, O, G)
        torch.cuda.synchronize()
        return out.float().cpu().numpy().ravel()

    x = np.array([[0.1 * d + 0.5 * v for d in range(64)] for v in range(3)], np.float32).ravel()
    assert np.abs(rt(x, 64, 0, 16) - x).max() <= 0.15
    x = np.array([0.01 * (i % 64) for i in range(128)], np.float32)
    for v in range(2):
        for k, ch in enumerate([3, 17, 33, 55]):
            x[v * 64 + ch] = 50.0 + k + v
    assert np.abs(rt(x, 64, 4, 16) - x).max() <= 0.1
    assert np.abs(rt(np.full(32, 2.5, np.float32), 32, 0, 16) - 2.5).max() <= 1e-2


def test_vector_codec_unsupported_params_leave_output_untouched():
    """test_kivi_roundtrip.cpp:207-229: head_dim 256 is refused, sentinel stays."""
    stride = tla.kivi_compressed_bytes(256, 0, 16)
    rec = torch.full((stride,), 0xAB, dtype=torch.uint8, device="cuda")
    x = torch.ones(1, 256, dtype=torch.float16, device="cuda")
    with pytest.raises(tla.TLError):
        tla.kivi_compress(x, rec, 1, 256, 0, 16)
    torch.cuda.synchronize()
    assert (rec.cpu().numpy() == 0xAB).all()


# ---------------------------------------------------------------------------
# paged KIVI
# ---------------------------------------------------------------------------

class KiviCase:
    """fp16 pools for the given lengths plus a page table over a page pool."""

    def __init__(self, seed, lens, H=32, n_kv=8, R=128, outliers=4, extra_blocks=4, bits=4, BS=16):
        self.lens = np.asarray(lens, np.int32)
        self.R = R
        self.bits = bits
        self.BS = BS
        self.page_bytes = orc.kivi_page_bytes(bits)
        S, D = len(lens), 128
        self.case = inputs.make_paged_case(seed, S, H, n_kv, D, BS,
                                           [L + extra_blocks * BS for L in lens], orc.F32)
        rng = np.random.default_rng(seed + 1)
        # outlier K channels per kv head scaled x8
        for h in range(n_kv):
            ch = rng.choice(D, size=outliers, replace=False)
            self.case.k_cache[:, h, ch, :] *= 8
        self.k = inputs.encode(self.case.k_cache, orc.F16)
        self.v = inputs.encode(self.case.v_cache, orc.F16)
        self.q = inputs.encode(orc.bits_to_f32(self.case.q, orc.F32), orc.F16)
        self.tables = self.case.tables
        self.n_kv, self.H, self.S = n_kv, H, S
        max_pages = max(1, (int(self.lens.max()) + extra_blocks * BS) // 32 + 1)
        self.num_pages = S * max_pages + 3
        perm = rng.permutation(self.num_pages).astype(np.int32)
        self.page_tables = perm[: S * max_pages].reshape(S, max_pages).copy()
        self.scale = 1 / math.sqrt(D)

    def oracle_pages(self, lens=None):
        pages = np.zeros((self.num_pages, self.n_kv, self.page_bytes), np.uint8)
        orc.kivi_build_pages(self.k, self.v, self.tables, self.lens if lens is None else lens, self.R,
                             pages, self.page_tables, self.bits)
        return pages

    def desc(self, qd, kd, btd, ptd, partition_pages=0, gqa=tla.GQA_GROUPED):
        return tla.make_kivi_desc(qd, kd, btd, ptd, self.num_pages, self.n_kv, self.scale,
                                  residual_length=self.R, gqa_map=gqa,
                                  partition_pages=partition_pages, bits=self.bits)


def _used_pages(kc, lens):
    used = set()
    for s, L in enumerate(lens):
        for p in range(orc.kivi_quantized_len(int(L), kc.R) // 32):
            used.add(int(kc.page_tables[s, p]))
    return sorted(used)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("R", [128, 0, 40])
def test_build_pages_bit_exact(R, bits):
    kc = KiviCase(51, [300, 1000, 161, 159, 0, 4096], R=R, bits=bits)
    want = kc.oracle_pages()
    qd, kd, vd = dev(kc.q, orc.F16), dev(kc.k, orc.F16), dev(kc.v, orc.F16)
    btd, sld, ptd = dev(kc.tables), dev(kc.lens), dev(kc.page_tables)
    pages = torch.zeros(kc.num_pages, kc.n_kv, kc.page_bytes, dtype=torch.uint8, device="cuda")
    print(f"case build pages R={R} bits={bits}", flush=True)
    tla.kivi_build_pages(kc.desc(qd, kd, btd, ptd), kd, vd, btd, sld, ptd, pages, int(kc.lens.max()))
    torch.cuda.synchronize()
    got = pages.cpu().numpy()
    used = _used_pages(kc, kc.lens)
    assert used, "case builds no page"
    assert np.array_equal(got[used], want[used])
    unused = sorted(set(range(kc.num_pages)) - set(used))
    assert (got[unused] == 0).all()


@pytest.mark.parametrize("bits", [4, 8])
def test_append_quantises_on_page_boundaries(bits):
    """Append one token per step for 70 steps; pages and the fp16 pool match
    a rebuild from the final pool, and pages appear exactly when Lq grows."""
    start = np.array([150, 159, 160, 191, 200], np.int32)
    steps = 70
    kc = KiviCase(52, start + steps, extra_blocks=1, bits=bits)
    print(f"case kivi append bits={bits}", flush=True)
    qd, kd, vd = dev(kc.q, orc.F16), dev(kc.k, orc.F16), dev(kc.v, orc.F16)
    btd, ptd = dev(kc.tables), dev(kc.page_tables)
    pages = torch.zeros(kc.num_pages, kc.n_kv, kc.page_bytes, dtype=torch.uint8, device="cuda")
    desc = kc.desc(qd, kd, btd, ptd)
    tla.kivi_build_pages(desc, kd, vd, btd, dev(start), ptd, pages, int(start.max()))
    rng = np.random.default_rng(9)
    lens = start.copy()
    k_host, v_host = kc.k.copy(), kc.v.copy()
    for _ in range(steps):
        lens = lens + 1
        pos = lens - 1
        slots = (kc.tables[np.arange(kc.S), pos // 16] * 16 + pos % 16).astype(np.int32)
        knew = inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16)
        vnew = inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16)
        tla.kivi_append(desc, dev(knew, orc.F16), dev(vnew, orc.F16), kd, vd, dev(slots), btd,
                        dev(lens), ptd, pages)
        orc.reshape_and_cache(knew, vnew, k_host, v_host, slots)
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(kd), k_host) and np.array_equal(host_bits(vd), v_host)
    kc.k, kc.v = k_host, v_host
    want = kc.oracle_pages(lens)
    used = _used_pages(kc, lens)
    got = pages.cpu().numpy()
    assert np.array_equal(got[used], want[used])


def _run_decode(kc, pages_np, partition_pages=0, gqa=tla.GQA_GROUPED):
    qd, kd, vd = dev(kc.q, orc.F16), dev(kc.k, orc.F16), dev(kc.v, orc.F16)
    btd, sld, ptd = dev(kc.tables), dev(kc.lens), dev(kc.page_tables)
    pages = torch.from_numpy(pages_np).cuda()
    desc = kc.desc(qd, kd, btd, ptd, partition_pages, gqa)
    max_ctx = int(kc.lens.max())
    ws = torch.empty(max(16, tla.kivi_workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
    out = torch.full_like(qd, float("nan"))
    tla.kivi_paged_attention_decode(desc, out, qd, pages, ptd, kd, vd, btd, sld, max_ctx, ws)
    torch.cuda.synchronize()
    return out


def _kivi_ref(kc, pages_np, gqa=orc.GROUPED):
    return orc.kivi_paged_attention(kc.q, orc.F16, pages_np, kc.page_tables, kc.k, kc.v, kc.tables,
                                    kc.lens, kc.n_kv, kc.R, kc.scale, gqa, kc.bits)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("pp", [-1, 0, 4, 1])
def test_kivi_decode_matches_oracle(pp, bits):
    kc = KiviCase(53, [4096, 1000, 161, 159, 0, 1, 2047, 3000], bits=bits)
    pages = kc.oracle_pages()
    print(f"case kivi decode pp={pp} bits={bits}", flush=True)
    assert_close(_run_decode(kc, pages, pp), _kivi_ref(kc, pages), orc.F16, ATOL_KIVI, f"pp={pp} bits={bits}")


@pytest.mark.parametrize("H,n_kv", [(16, 8), (64, 8), (8, 8)])
@pytest.mark.parametrize("gqa", [tla.GQA_GROUPED, tla.GQA_MODULO])
def test_kivi_decode_group_sizes(H, n_kv, gqa):
    kc = KiviCase(54, [700, 300, 2000], H=H, n_kv=n_kv)
    pages = kc.oracle_pages()
    print(f"case kivi H={H} n_kv={n_kv} gqa={gqa}", flush=True)
    assert_close(_run_decode(kc, pages, 0, gqa), _kivi_ref(kc, pages, gqa), orc.F16, ATOL_KIVI,
                 f"H={H}")


def _punch_holes(kc):
    """Holes of every kind on a KiviCase with lengths [4096, 1000, 300, 161,
    2047, 700] (R = 128): block-table holes in the fp16 window (one on the
    newest token), a block hole inside a page's range (the page then holds
    quantised zeros), page-table entries that are negative or past the page
    pool, and a sequence whose every page is a hole."""
    t = kc.tables
    t[0, (4096 - 50) // 16] = -1            # window of sequence 0 (Lq = 3968)
    t[1, (1000 - 1) // 16] = -1             # the newest token's block of sequence 1
    t[2, 3] = -1                            # inside page 1 of sequence 2 (Lq = 160)
    t[4, (2047 - 140) // 16] = -1           # a window block of sequence 4 (Lq = 1888)
    pt = kc.page_tables
    pt[0, 7] = -1
    pt[0, 100] = kc.num_pages               # past the pool: a hole
    pt[4, 0] = -1
    pt[5, :] = -1                           # sequence 5: every page a hole (Lq = 544)


@pytest.mark.parametrize("pp,bits", [(0, 4), (4, 4), (-1, 4), (4, 8)])
def test_kivi_decode_table_and_page_holes(pp, bits):
    """Holes in the block table (fp16 window) and the page table are skipped
    by the decode, as the oracle skips them; a hole inside a page's block
    range only zeroes the tokens the page was built from."""
    kc = KiviCase(59, [4096, 1000, 300, 161, 2047, 700], bits=bits)
    _punch_holes(kc)
    pages = kc.oracle_pages()
    print(f"case kivi holes pp={pp} bits={bits}", flush=True)
    assert_close(_run_decode(kc, pages, pp), _kivi_ref(kc, pages), orc.F16, ATOL_KIVI, f"holes pp={pp}")


def test_kivi_split_k_page_table_narrower_than_sequence():
    """A page table with fewer columns than a sequence has pages: the pages
    past its width are dropped by the decode and by the log-sum-exp merge
    alike (the merge counts the partitions the decode wrote, not those of
    the full length); the workspace starts as finite values a merge of
    unwritten partitions would pick up."""
    kc = KiviCase(62, [4096, 3000, 700, 161])
    kc.page_tables = np.ascontiguousarray(kc.page_tables[:, :20])
    pages = kc.oracle_pages()
    qd, kd, vd = dev(kc.q, orc.F16), dev(kc.k, orc.F16), dev(kc.v, orc.F16)
    btd, sld, ptd = dev(kc.tables), dev(kc.lens), dev(kc.page_tables)
    desc = kc.desc(qd, kd, btd, ptd, 4)
    max_ctx = int(kc.lens.max())
    nbytes = tla.kivi_workspace_bytes(desc, max_ctx)
    assert nbytes > 0 and nbytes % 4 == 0
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    ws.view(torch.float32).fill_(1.0)
    out = torch.full_like(qd, float("nan"))
    print("case kivi narrow page table pp=4", flush=True)
    tla.kivi_paged_attention_decode(desc, out, qd, torch.from_numpy(pages).cuda(), ptd, kd, vd, btd, sld,
                                    max_ctx, ws)
    torch.cuda.synchronize()
    assert_close(out, _kivi_ref(kc, pages), orc.F16, ATOL_KIVI, "narrow page table")


@pytest.mark.parametrize("bits", [4, 8])
def test_build_pages_with_holes_bit_exact(bits):
    """The GPU page build skips page-table holes (negative or past the pool)
    and quantises a block-table hole as zeros, byte for byte as the oracle."""
    kc = KiviCase(60, [4096, 1000, 300, 161, 2047, 700], bits=bits)
    _punch_holes(kc)
    want = kc.oracle_pages()
    qd, kd, vd = dev(kc.q, orc.F16), dev(kc.k, orc.F16), dev(kc.v, orc.F16)
    btd, sld, ptd = dev(kc.tables), dev(kc.lens), dev(kc.page_tables)
    pages = torch.zeros(kc.num_pages, kc.n_kv, kc.page_bytes, dtype=torch.uint8, device="cuda")
    print("case build pages with holes", flush=True)
    tla.kivi_build_pages(kc.desc(qd, kd, btd, ptd), kd, vd, btd, sld, ptd, pages, int(kc.lens.max()))
    torch.cuda.synchronize()
    assert np.array_equal(pages.cpu().numpy(), want)


@pytest.mark.parametrize("H,pp,bits", [(32, 0, 4), (64, 4, 4), (32, 0, 8), (64, 4, 8)])
def test_kivi_decode_step_matches_oracle_each_step(H, pp, bits):
    """The fused tl_kivi_decode_step checked against the oracle itself at
    every step: the host pools receive each token through
    orc.reshape_and_cache, the pages are rebuilt by orc.kivi_build_pages at
    the step's lengths and the expected output is orc.kivi_paged_attention.
    Sequences complete pages during the run; sequence 0's first page and a
    window block of sequence 5 are holes."""
    start = np.array([150, 159, 160, 191, 33, 1000], np.int32)
    steps = 36
    kc = KiviCase(61, start + steps, H=H, extra_blocks=1, bits=bits)
    kc.page_tables[0, 0] = -1
    kc.tables[5, (1000 - 60) // 16] = -1
    qd, kd, vd = dev(kc.q, orc.F16), dev(kc.k, orc.F16), dev(kc.v, orc.F16)
    btd, ptd = dev(kc.tables), dev(kc.page_tables)
    pages = torch.zeros(kc.num_pages, kc.n_kv, kc.page_bytes, dtype=torch.uint8, device="cuda")
    desc = kc.desc(qd, kd, btd, ptd, pp)
    tla.kivi_build_pages(desc, kd, vd, btd, dev(start), ptd, pages, int(start.max()))
    rng = np.random.default_rng(12)
    max_ctx = int(start.max()) + steps
    ws = torch.empty(max(16, tla.kivi_workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
    lens = start.copy()
    k_host, v_host = kc.k.copy(), kc.v.copy()
    print(f"case kivi step vs oracle H={H} pp={pp} bits={bits}", flush=True)
    for step in range(steps):
        lens = lens + 1
        pos = lens - 1
        slots = (kc.tables[np.arange(kc.S), pos // 16] * 16 + pos % 16).astype(np.int32)
        knew = inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16)
        vnew = inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16)
        out = torch.full_like(qd, float("nan"))
        tla.kivi_decode_step(desc, out, qd, dev(knew, orc.F16), dev(vnew, orc.F16), dev(slots), pages, ptd,
                             kd, vd, btd, dev(lens), max_ctx, ws)
        torch.cuda.synchronize()
        orc.reshape_and_cache(knew, vnew, k_host, v_host, slots)
        kc.k, kc.v, kc.lens = k_host, v_host, lens
        want_pages = kc.oracle_pages()
        want = _kivi_ref(kc, want_pages)
        assert_close(out, want, orc.F16, ATOL_KIVI, f"step {step}")
    used = _used_pages(kc, lens)
    used = [p for p in used if p >= 0]
    assert np.array_equal(pages.cpu().numpy()[used], want_pages[used])


def _oracle_rotate(q, knew, vnew, pos, cos_t, sin_t, style):
    """The oracle's RoPE of q [S, H, 128] and of the new keys at pos (a
    position past the tables leaves the rows unrotated), by way of a scratch
    pool that holds token t in slot t."""
    S, n_kv, D = knew.shape
    q_out = q.copy()
    nb = (S + 15) // 16
    kpool = np.zeros((nb, n_kv, D, 16), np.uint16)
    vpool = np.zeros_like(kpool)
    slots = np.arange(S, dtype=np.int32)
    orc.reshape_and_cache(knew, vnew, kpool, vpool, slots)
    orc.rope_reshape_and_cache(q, q_out, knew, vnew, kpool, vpool, slots, pos, cos_t, sin_t, orc.F16, style)
    k_rot = np.ascontiguousarray(kpool.transpose(0, 3, 1, 2).reshape(nb * 16, n_kv, D)[:S])
    return q_out, k_rot


@pytest.mark.parametrize("style,bits", [(tla.ROPE_ADJACENT, 4), (tla.ROPE_HALVES, 8), (tla.ROPE_ADJACENT, 8)])
def test_kivi_rope_step_matches_oracle_each_step(style, bits):
    """tl_kivi_rope_decode_step (RoPE of q and the new keys, then the fused
    step on the rotated rows) against the oracle at every step: the
    oracle's RoPE, the rotated key into the host pools, the pages rebuilt
    and orc.kivi_paged_attention with the rotated q.  Sequence 5 runs past
    the 1024-position tables halfway (those tokens stay unrotated); pages
    complete during the run.  At the end the pools and pages are the
    oracle's bit for bit."""
    from test_oracle import rope_tables
    start = np.array([150, 159, 160, 191, 33, 1000], np.int32)
    steps = 36
    kc = KiviCase(71, start + steps, H=32, extra_blocks=1, bits=bits)
    cos_t, sin_t = rope_tables(1024, 128)
    q_base = kc.q.copy()
    qd, kd, vd = dev(kc.q, orc.F16), dev(kc.k, orc.F16), dev(kc.v, orc.F16)
    btd, ptd = dev(kc.tables), dev(kc.page_tables)
    pages = torch.zeros(kc.num_pages, kc.n_kv, kc.page_bytes, dtype=torch.uint8, device="cuda")
    desc = kc.desc(qd, kd, btd, ptd, 0)
    tla.kivi_build_pages(desc, kd, vd, btd, dev(start), ptd, pages, int(start.max()))
    rng = np.random.default_rng(13)
    max_ctx = int(start.max()) + steps
    ws = torch.empty(tla.kivi_rope_step_workspace_bytes(desc, max_ctx), dtype=torch.uint8, device="cuda")
    cos_d, sin_d = dev(cos_t), dev(sin_t)
    lens = start.copy()
    k_host, v_host = kc.k.copy(), kc.v.copy()
    print(f"case kivi rope step vs oracle style={style} bits={bits}", flush=True)
    for step in range(steps):
        lens = lens + 1
        pos = (lens - 1).astype(np.int32)
        slots = (kc.tables[np.arange(kc.S), pos // 16] * 16 + pos % 16).astype(np.int32)
        knew = inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16)
        vnew = inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16)
        out = torch.full_like(qd, float("nan"))
        tla.kivi_rope_decode_step(desc, out, qd, dev(knew, orc.F16), dev(vnew, orc.F16), dev(pos), cos_d, sin_d,
                                  style, dev(slots), pages, ptd, kd, vd, btd, dev(lens), max_ctx, ws)
        torch.cuda.synchronize()
        q_rot, k_rot = _oracle_rotate(q_base, knew, vnew, pos, cos_t, sin_t, style)
        orc.reshape_and_cache(k_rot, vnew, k_host, v_host, slots)
        kc.q, kc.k, kc.v, kc.lens = q_rot, k_host, v_host, lens
        want_pages = kc.oracle_pages()
        assert_close(out, _kivi_ref(kc, want_pages), orc.F16, ATOL_KIVI, f"step {step}")
    assert np.array_equal(host_bits(kd), k_host) and np.array_equal(host_bits(vd), v_host)
    used = [p for p in _used_pages(kc, lens) if p >= 0]
    assert np.array_equal(pages.cpu().numpy()[used], want_pages[used])


@pytest.mark.parametrize("style,bits,pp", [(tla.ROPE_ADJACENT, 4, 0), (tla.ROPE_HALVES, 4, -1),
                                           (tla.ROPE_HALVES, 8, 4), (tla.ROPE_ADJACENT, 8, 1)])
def test_kivi_pre_rope_decode_matches_oracle(style, bits, pp):
    """Keys held before RoPE (tl_kivi_paged_attention_decode_pre_rope): each
    page key rotated after its dequantisation and each window key as read,
    at its token position, against the oracle's attention on the rotated
    keys; a page and a window block are holes.  The same descriptor through
    the standard entry point is refused, and so are tables that do not cover
    every position (2048 positions for a 4096-token sequence)."""
    from test_oracle import rope_tables
    kc = KiviCase(57, [4096, 1000, 161, 159, 0, 1, 2047, 3000], bits=bits)
    kc.page_tables[1, 3] = -1
    kc.tables[6, (2047 - 60) // 16] = -1
    pages_np = kc.oracle_pages()
    cos_t, sin_t = rope_tables(4096, 128)
    qd, kd, vd = dev(kc.q, orc.F16), dev(kc.k, orc.F16), dev(kc.v, orc.F16)
    btd, sld, ptd = dev(kc.tables), dev(kc.lens), dev(kc.page_tables)
    pages = torch.from_numpy(pages_np).cuda()
    desc = kc.desc(qd, kd, btd, ptd, pp)
    desc.pre_rope_keys = 1
    max_ctx = int(kc.lens.max())
    ws = torch.empty(max(16, tla.kivi_workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
    out = torch.full_like(qd, float("nan"))
    print(f"case kivi pre-rope decode style={style} bits={bits} pp={pp}", flush=True)
    tla.kivi_paged_attention_decode_pre_rope(desc, out, qd, pages, ptd, kd, vd, btd, sld, max_ctx, dev(cos_t),
                                             dev(sin_t), style, ws)
    torch.cuda.synchronize()
    want = orc.kivi_paged_attention(kc.q, orc.F16, pages_np, kc.page_tables, kc.k, kc.v, kc.tables, kc.lens,
                                    kc.n_kv, kc.R, kc.scale, orc.GROUPED, bits, pre_rope=(cos_t, sin_t, style))
    assert_close(out, want, orc.F16, ATOL_KIVI, f"style={style} bits={bits} pp={pp}")
    with pytest.raises(tla.TLError):
        tla.kivi_paged_attention_decode(desc, out, qd, pages, ptd, kd, vd, btd, sld, max_ctx, ws)
    short_c, short_s = dev(cos_t[:2048].copy()), dev(sin_t[:2048].copy())
    with pytest.raises(tla.TLError):
        tla.kivi_paged_attention_decode_pre_rope(desc, out, qd, pages, ptd, kd, vd, btd, sld, max_ctx, short_c,
                                                 short_s, style, ws)


@pytest.mark.parametrize("style", [tla.ROPE_ADJACENT, tla.ROPE_HALVES])
@pytest.mark.parametrize("bits", [4, 8])
def test_kivi_pre_rope_long_single_pass(style, bits):
    """A workgroup holds the rotations of at most 160 (INT4) / 144 (INT8)
    pages in LDS, so a single pass asked for over sequences of 180, 135 and
    114 pages runs in two partitions (at INT8 the 135-page sequence fits one
    partition, the 180-page one spans both), against the oracle; a page in
    each partition is a hole."""
    from test_oracle import rope_tables
    kc = KiviCase(58, [5900, 4460, 3800, 900], bits=bits)
    kc.page_tables[0, 140] = -1
    kc.page_tables[0, 170] = -1
    pages_np = kc.oracle_pages()
    cos_t, sin_t = rope_tables(5900, 128)
    qd, kd, vd = dev(kc.q, orc.F16), dev(kc.k, orc.F16), dev(kc.v, orc.F16)
    btd, sld, ptd = dev(kc.tables), dev(kc.lens), dev(kc.page_tables)
    pages = torch.from_numpy(pages_np).cuda()
    desc = kc.desc(qd, kd, btd, ptd, -1)
    desc.pre_rope_keys = 1
    max_ctx = int(kc.lens.max())
    ws = torch.empty(max(16, tla.kivi_workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
    out = torch.full_like(qd, float("nan"))
    print(f"case kivi pre-rope long single pass style={style} bits={bits}", flush=True)
    tla.kivi_paged_attention_decode_pre_rope(desc, out, qd, pages, ptd, kd, vd, btd, sld, max_ctx, dev(cos_t),
                                             dev(sin_t), style, ws)
    torch.cuda.synchronize()
    want = orc.kivi_paged_attention(kc.q, orc.F16, pages_np, kc.page_tables, kc.k, kc.v, kc.tables, kc.lens,
                                    kc.n_kv, kc.R, kc.scale, orc.GROUPED, bits, pre_rope=(cos_t, sin_t, style))
    assert_close(out, want, orc.F16, ATOL_KIVI, f"style={style} bits={bits} long single pass")


@pytest.mark.parametrize("H,n_kv", [(16, 8), (64, 8), (8, 8)])
@pytest.mark.parametrize("gqa", [tla.GQA_GROUPED, tla.GQA_MODULO])
def test_kivi_pre_rope_decode_group_sizes(H, n_kv, gqa):
    """Keys held before RoPE with GQA groups of 2, 8 and 1 under both head
    maps (halves style, INT4, the library's partition plan)."""
    from test_oracle import rope_tables
    kc = KiviCase(58, [700, 300, 2000], H=H, n_kv=n_kv)
    pages_np = kc.oracle_pages()
    cos_t, sin_t = rope_tables(4096, 128)
    qd, kd, vd = dev(kc.q, orc.F16), dev(kc.k, orc.F16), dev(kc.v, orc.F16)
    btd, sld, ptd = dev(kc.tables), dev(kc.lens), dev(kc.page_tables)
    desc = kc.desc(qd, kd, btd, ptd, 0, gqa)
    desc.pre_rope_keys = 1
    max_ctx = int(kc.lens.max())
    ws = torch.empty(max(16, tla.kivi_workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
    out = torch.full_like(qd, float("nan"))
    print(f"case kivi pre-rope H={H} n_kv={n_kv} gqa={gqa}", flush=True)
    tla.kivi_paged_attention_decode_pre_rope(desc, out, qd, torch.from_numpy(pages_np).cuda(), ptd, kd, vd, btd, sld,
                                             max_ctx, dev(cos_t), dev(sin_t), tla.ROPE_HALVES, ws)
    torch.cuda.synchronize()
    omap = orc.GROUPED if gqa == tla.GQA_GROUPED else orc.MODULO
    want = orc.kivi_paged_attention(kc.q, orc.F16, pages_np, kc.page_tables, kc.k, kc.v, kc.tables, kc.lens,
                                    kc.n_kv, kc.R, kc.scale, omap, kc.bits, pre_rope=(cos_t, sin_t, tla.ROPE_HALVES))
    assert_close(out, want, orc.F16, ATOL_KIVI, f"H={H} gqa={gqa}")


@pytest.mark.parametrize("style,bits,through_rope_step", [(tla.ROPE_ADJACENT, 4, True), (tla.ROPE_HALVES, 8, True),
                                                          (tla.ROPE_HALVES, 4, False)])
def test_kivi_pre_rope_step_matches_oracle_each_step(style, bits, through_rope_step):
    """Keys held before RoPE through the fused step, checked against the
    oracle at every step.  Through tl_kivi_rope_decode_step with the
    descriptor's pre_rope_keys set, q is rotated at position seq_lens - 1 and
    the new key goes to the pool as given; through
    tl_kivi_decode_step_pre_rope, q is taken as given.  The host pools take
    the unrotated keys, the pages are rebuilt from them, and the expected
    output is the oracle's attention with every key rotated at its position.
    Pages complete during the run.  At the end the pools and pages are the
    oracle's bit for bit (unrotated keys)."""
    from test_oracle import rope_tables
    start = np.array([150, 159, 160, 191, 33, 1000], np.int32)
    steps = 36
    kc = KiviCase(73, start + steps, H=32, extra_blocks=1, bits=bits)
    cos_t, sin_t = rope_tables(1040, 128)
    q_base = kc.q.copy()
    qd, kd, vd = dev(kc.q, orc.F16), dev(kc.k, orc.F16), dev(kc.v, orc.F16)
    btd, ptd = dev(kc.tables), dev(kc.page_tables)
    pages = torch.zeros(kc.num_pages, kc.n_kv, kc.page_bytes, dtype=torch.uint8, device="cuda")
    desc = kc.desc(qd, kd, btd, ptd, 0)
    tla.kivi_build_pages(desc, kd, vd, btd, dev(start), ptd, pages, int(start.max()))
    tla.kivi_apply_config(desc, bits=bits, residual_length=kc.R, pre_rope_keys=True)
    rng = np.random.default_rng(15)
    max_ctx = int(start.max()) + steps
    ws = torch.empty(max(16, tla.kivi_rope_step_workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
    cos_d, sin_d = dev(cos_t), dev(sin_t)
    lens = start.copy()
    k_host, v_host = kc.k.copy(), kc.v.copy()
    print(f"case kivi pre-rope step style={style} bits={bits} rope_step={through_rope_step}", flush=True)
    for step in range(steps):
        lens = lens + 1
        pos = (lens - 1).astype(np.int32)
        slots = (kc.tables[np.arange(kc.S), pos // 16] * 16 + pos % 16).astype(np.int32)
        knew = inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16)
        vnew = inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16)
        out = torch.full_like(qd, float("nan"))
        if through_rope_step:
            tla.kivi_rope_decode_step(desc, out, qd, dev(knew, orc.F16), dev(vnew, orc.F16), dev(pos), cos_d, sin_d,
                                      style, dev(slots), pages, ptd, kd, vd, btd, dev(lens), max_ctx, ws)
            q_use, _ = _oracle_rotate(q_base, knew, vnew, pos, cos_t, sin_t, style)
        else:
            tla.kivi_decode_step_pre_rope(desc, out, qd, dev(knew, orc.F16), dev(vnew, orc.F16), dev(slots), pages,
                                          ptd, kd, vd, btd, dev(lens), max_ctx, cos_d, sin_d, style, ws)
            q_use = q_base
        torch.cuda.synchronize()
        orc.reshape_and_cache(knew, vnew, k_host, v_host, slots)
        kc.k, kc.v, kc.lens = k_host, v_host, lens
        want_pages = kc.oracle_pages()
        want = orc.kivi_paged_attention(q_use, orc.F16, want_pages, kc.page_tables, kc.k, kc.v, kc.tables, kc.lens,
                                        kc.n_kv, kc.R, kc.scale, orc.GROUPED, bits, pre_rope=(cos_t, sin_t, style))
        assert_close(out, want, orc.F16, ATOL_KIVI, f"step {step}")
    assert np.array_equal(host_bits(kd), k_host) and np.array_equal(host_bits(vd), v_host)
    used = [p for p in _used_pages(kc, lens) if p >= 0]
    assert np.array_equal(pages.cpu().numpy()[used], want_pages[used])


def test_kivi_step_full_batch_mixed_lengths():
    """The benchmark's KIVI step at full size: batch 64, 32/8 heads,
    sequence s at 4096 + s mod 32 tokens, R = 128, one fused step (sequences
    31 and 63 complete a page in it).  The pages of every sequence are the
    oracle's bit for bit; the outputs of 16 sequences, those two included,
    match the oracle."""
    start = np.array([4096 + s % 32 for s in range(64)], np.int32)
    kc = KiviCase(81, start + 1, H=32, extra_blocks=1)
    qd, kd, vd = dev(kc.q, orc.F16), dev(kc.k, orc.F16), dev(kc.v, orc.F16)
    btd, ptd = dev(kc.tables), dev(kc.page_tables)
    pages = torch.zeros(kc.num_pages, kc.n_kv, kc.page_bytes, dtype=torch.uint8, device="cuda")
    desc = kc.desc(qd, kd, btd, ptd, 0)
    tla.kivi_build_pages(desc, kd, vd, btd, dev(start), ptd, pages, int(start.max()))
    rng = np.random.default_rng(14)
    lens = start + 1
    pos = start
    slots = (kc.tables[np.arange(kc.S), pos // 16] * 16 + pos % 16).astype(np.int32)
    knew = inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16)
    vnew = inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16)
    max_ctx = int(lens.max())
    ws = torch.empty(max(16, tla.kivi_workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
    out = torch.full_like(qd, float("nan"))
    print("case kivi step full batch, mixed lengths", flush=True)
    tla.kivi_decode_step(desc, out, qd, dev(knew, orc.F16), dev(vnew, orc.F16), dev(slots), pages, ptd, kd, vd, btd,
                         dev(lens), max_ctx, ws)
    torch.cuda.synchronize()
    orc.reshape_and_cache(knew, vnew, kc.k, kc.v, slots)
    kc.lens = lens
    want_pages = kc.oracle_pages()
    used = [p for p in _used_pages(kc, lens) if p >= 0]
    assert np.array_equal(pages.cpu().numpy()[used], want_pages[used])
    assert np.array_equal(host_bits(kd), kc.k) and np.array_equal(host_bits(vd), kc.v)
    sub = np.array([0, 1, 5, 9, 15, 16, 22, 30, 31, 32, 40, 47, 50, 58, 62, 63])
    want = orc.kivi_paged_attention(np.ascontiguousarray(kc.q[sub]), orc.F16, want_pages,
                                    np.ascontiguousarray(kc.page_tables[sub]), kc.k, kc.v,
                                    np.ascontiguousarray(kc.tables[sub]), np.ascontiguousarray(lens[sub]),
                                    kc.n_kv, kc.R, kc.scale, orc.GROUPED, kc.bits)
    assert_close(out[torch.from_numpy(sub).cuda()], want, orc.F16, ATOL_KIVI, "full batch")
    assert torch.isfinite(out).all()


def test_kivi_decode_residual_zero_and_nan_slots():
    """R = 0 (every whole page quantised) and NaN in unused fp16 slots."""
    kc = KiviCase(55, [96, 100, 33], R=0)
    for s, L in enumerate(kc.lens):
        last = kc.tables[s, (L - 1) // 16]
        kc.v[last, :, :, L % 16 or 16:] = 0x7E00
        kc.k[last, :, :, L % 16 or 16:] = 0x7E00
    pages = kc.oracle_pages()
    assert_close(_run_decode(kc, pages, -1), _kivi_ref(kc, pages), orc.F16, ATOL_KIVI, "R=0")


@pytest.mark.parametrize("fused", [False, True])
def test_kivi_step_graph_replay_matches_eager(fused):
    """One append + decode step (two calls, or the fused tl_kivi_decode_step)
    captured in a HIP graph and replayed three times, with eager work between
    replays: every replay matches the eager step bit for bit (the append is
    idempotent: same token, same slot).  Sequence 1 (159 -> 160 tokens)
    completes a page in the step."""
    start = np.array([700, 159, 2000, 129], np.int32)
    kc = KiviCase(57, start + 1, extra_blocks=1)
    qd, kd, vd = dev(kc.q, orc.F16), dev(kc.k, orc.F16), dev(kc.v, orc.F16)
    btd, ptd = dev(kc.tables), dev(kc.page_tables)
    pages = torch.zeros(kc.num_pages, kc.n_kv, kc.page_bytes, dtype=torch.uint8, device="cuda")
    desc = kc.desc(qd, kd, btd, ptd)
    tla.kivi_build_pages(desc, kd, vd, btd, dev(start), ptd, pages, int(start.max()))
    lens = start + 1
    pos = lens - 1
    slots = dev((kc.tables[np.arange(kc.S), pos // 16] * 16 + pos % 16).astype(np.int32))
    rng = np.random.default_rng(10)
    knew = dev(inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16), orc.F16)
    vnew = dev(inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16), orc.F16)
    sld = dev(lens)
    max_ctx = int(lens.max())
    ws = torch.empty(max(16, tla.kivi_workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
    out = torch.zeros_like(qd)

    def step(stream):
        if fused:
            tla.kivi_decode_step(desc, out, qd, knew, vnew, slots, pages, ptd, kd, vd, btd, sld, max_ctx, ws,
                                 stream)
            return
        tla.kivi_append(desc, knew, vnew, kd, vd, slots, btd, sld, ptd, pages, stream)
        tla.kivi_paged_attention_decode(desc, out, qd, pages, ptd, kd, vd, btd, sld, max_ctx, ws, stream)

    print(f"case kivi graph replay fused={fused}", flush=True)
    step(torch.cuda.current_stream())
    torch.cuda.synchronize()
    eager, eager_pages = out.clone(), pages.clone()
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=cap):
        step(cap)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        assert torch.equal(pages, eager_pages)
        step(torch.cuda.current_stream())            # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


@pytest.mark.parametrize("H,R,pp,bits", [(32, 128, 0, 4), (32, 0, 0, 4), (64, 128, 0, 4), (32, 128, 4, 4),
                                         (64, 0, 4, 4), (32, 20, 0, 4), (32, 128, 0, 8), (64, 0, 4, 8)])
def test_decode_step_equals_append_then_decode(H, R, pp, bits):
    """tl_kivi_decode_step gives the bytes of tl_kivi_append followed by
    tl_kivi_paged_attention_decode, over 40 steps that complete pages."""
    start = np.array([150, 159, 160, 191, 33, 1000], np.int32)
    steps = 40
    runs = []
    for fused in (False, True):
        kc = KiviCase(58, start + steps, H=H, R=R, extra_blocks=1, bits=bits)
        qd, kd, vd = dev(kc.q, orc.F16), dev(kc.k, orc.F16), dev(kc.v, orc.F16)
        btd, ptd = dev(kc.tables), dev(kc.page_tables)
        pages = torch.zeros(kc.num_pages, kc.n_kv, kc.page_bytes, dtype=torch.uint8, device="cuda")
        desc = kc.desc(qd, kd, btd, ptd, pp)
        tla.kivi_build_pages(desc, kd, vd, btd, dev(start), ptd, pages, int(start.max()))
        rng = np.random.default_rng(11)
        max_ctx = int(start.max()) + steps
        ws = torch.empty(max(16, tla.kivi_workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
        lens = start.copy()
        outs = []
        print(f"case kivi step H={H} R={R} pp={pp} bits={bits} fused={fused}", flush=True)
        for _ in range(steps):
            lens = lens + 1
            pos = lens - 1
            slots = dev((kc.tables[np.arange(kc.S), pos // 16] * 16 + pos % 16).astype(np.int32))
            knew = dev(inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16), orc.F16)
            vnew = dev(inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16), orc.F16)
            sld = dev(lens)
            out = torch.full_like(qd, float("nan"))
            if fused:
                tla.kivi_decode_step(desc, out, qd, knew, vnew, slots, pages, ptd, kd, vd, btd, sld, max_ctx, ws)
            else:
                tla.kivi_append(desc, knew, vnew, kd, vd, slots, btd, sld, ptd, pages)
                tla.kivi_paged_attention_decode(desc, out, qd, pages, ptd, kd, vd, btd, sld, max_ctx, ws)
            outs.append(out)
        torch.cuda.synchronize()
        runs.append((torch.stack(outs), pages.clone(), kd.clone(), vd.clone()))
    for a, b in zip(runs[0], runs[1]):
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))


@pytest.mark.parametrize("style,bits,pp", [(tla.ROPE_HALVES, 4, 0), (tla.ROPE_ADJACENT, 8, 4), (tla.ROPE_HALVES, 4, -1)])
def test_pre_rope_step_equals_append_then_pre_rope_decode(style, bits, pp):
    """Keys held before RoPE: tl_kivi_decode_step_pre_rope gives the bytes of
    tl_kivi_append followed by tl_kivi_paged_attention_decode_pre_rope
    (outputs, pages and pools), over 40 steps that complete pages."""
    from test_oracle import rope_tables
    start = np.array([150, 159, 160, 191, 33, 1000], np.int32)
    steps = 40
    cos_t, sin_t = rope_tables(1040, 128)
    runs = []
    for fused in (False, True):
        kc = KiviCase(59, start + steps, H=32, extra_blocks=1, bits=bits)
        qd, kd, vd = dev(kc.q, orc.F16), dev(kc.k, orc.F16), dev(kc.v, orc.F16)
        btd, ptd = dev(kc.tables), dev(kc.page_tables)
        cos_d, sin_d = dev(cos_t), dev(sin_t)
        pages = torch.zeros(kc.num_pages, kc.n_kv, kc.page_bytes, dtype=torch.uint8, device="cuda")
        desc = kc.desc(qd, kd, btd, ptd, pp)
        tla.kivi_build_pages(desc, kd, vd, btd, dev(start), ptd, pages, int(start.max()))
        desc.pre_rope_keys = 1
        rng = np.random.default_rng(12)
        max_ctx = int(start.max()) + steps
        ws = torch.empty(max(16, tla.kivi_workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
        lens = start.copy()
        outs = []
        print(f"case kivi pre-rope step equivalence style={style} bits={bits} pp={pp} fused={fused}", flush=True)
        for _ in range(steps):
            lens = lens + 1
            pos = lens - 1
            slots = dev((kc.tables[np.arange(kc.S), pos // 16] * 16 + pos % 16).astype(np.int32))
            knew = dev(inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16), orc.F16)
            vnew = dev(inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16), orc.F16)
            sld = dev(lens)
            out = torch.full_like(qd, float("nan"))
            if fused:
                tla.kivi_decode_step_pre_rope(desc, out, qd, knew, vnew, slots, pages, ptd, kd, vd, btd, sld, max_ctx,
                                              cos_d, sin_d, style, ws)
            else:
                tla.kivi_append(desc, knew, vnew, kd, vd, slots, btd, sld, ptd, pages)
                tla.kivi_paged_attention_decode_pre_rope(desc, out, qd, pages, ptd, kd, vd, btd, sld, max_ctx, cos_d,
                                                         sin_d, style, ws)
            outs.append(out)
        torch.cuda.synchronize()
        runs.append((torch.stack(outs), pages.clone(), kd.clone(), vd.clone()))
    for a, b in zip(runs[0], runs[1]):
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))


@pytest.mark.parametrize("through_rope_step", [False, True])
def test_pre_rope_step_graph_replay_matches_eager(through_rope_step):
    """Keys held before RoPE: the step (tl_kivi_decode_step_pre_rope, or
    tl_kivi_rope_decode_step with the flag: the q rotation launch, then the
    step) captured in a HIP graph and replayed three times with eager work
    between replays: every replay matches the eager step bit for bit.
    Sequence 1 (159 -> 160 tokens) completes a page in the step."""
    from test_oracle import rope_tables
    start = np.array([700, 159, 2000, 129], np.int32)
    kc = KiviCase(60, start + 1, extra_blocks=1)
    qd, kd, vd = dev(kc.q, orc.F16), dev(kc.k, orc.F16), dev(kc.v, orc.F16)
    btd, ptd = dev(kc.tables), dev(kc.page_tables)
    pages = torch.zeros(kc.num_pages, kc.n_kv, kc.page_bytes, dtype=torch.uint8, device="cuda")
    desc = kc.desc(qd, kd, btd, ptd)
    tla.kivi_build_pages(desc, kd, vd, btd, dev(start), ptd, pages, int(start.max()))
    desc.pre_rope_keys = 1
    cos_t, sin_t = rope_tables(4096, 128)
    cos_d, sin_d = dev(cos_t), dev(sin_t)
    lens = start + 1
    pos = lens - 1
    slots = dev((kc.tables[np.arange(kc.S), pos // 16] * 16 + pos % 16).astype(np.int32))
    posd = dev(pos.astype(np.int32))
    rng = np.random.default_rng(16)
    knew = dev(inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16), orc.F16)
    vnew = dev(inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16), orc.F16)
    sld = dev(lens)
    max_ctx = int(lens.max())
    ws = torch.empty(max(16, tla.kivi_rope_step_workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
    out = torch.zeros_like(qd)

    def step(stream):
        if through_rope_step:
            tla.kivi_rope_decode_step(desc, out, qd, knew, vnew, posd, cos_d, sin_d, tla.ROPE_HALVES, slots, pages, ptd,
                                      kd, vd, btd, sld, max_ctx, ws, stream)
        else:
            tla.kivi_decode_step_pre_rope(desc, out, qd, knew, vnew, slots, pages, ptd, kd, vd, btd, sld, max_ctx,
                                          cos_d, sin_d, tla.ROPE_HALVES, ws, stream)

    print(f"case kivi pre-rope graph replay rope_step={through_rope_step}", flush=True)
    step(torch.cuda.current_stream())
    torch.cuda.synchronize()
    eager, eager_pages = out.clone(), pages.clone()
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=cap):
        step(cap)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        assert torch.equal(pages, eager_pages)
        step(torch.cuda.current_stream())            # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


@pytest.mark.parametrize("BS", [8, 32, 64, 256])
def test_kivi_block_sizes_step_and_decode_against_oracle(BS):
    """The fp16 pool at block sizes other than 16 (any power of two 8..256):
    pages built bit-exact, the fused step against the oracle at every step
    (the window and the newest token read at that block size, the token
    stored into its block while the other slots keep their bytes: the pools
    are compared bit for bit at the end), then the two-launch decode under
    single pass and split-K, INT4 and INT8 pages.  A window block of
    sequence 3 is a hole."""
    start = np.array([150, 159, 190, 1000, 33, 700], np.int32)
    steps = 34
    for bits in (4, 8):
        kc = KiviCase(62 + BS + bits, start + steps, H=32, extra_blocks=1, bits=bits, BS=BS)
        hole_lb = (1000 - 60) // BS
        kc.tables[3, hole_lb] = -1
        qd, kd, vd = dev(kc.q, orc.F16), dev(kc.k, orc.F16), dev(kc.v, orc.F16)
        btd, ptd = dev(kc.tables), dev(kc.page_tables)
        pages = torch.zeros(kc.num_pages, kc.n_kv, kc.page_bytes, dtype=torch.uint8, device="cuda")
        desc = kc.desc(qd, kd, btd, ptd, 0)
        assert desc.block_size == BS
        print(f"case kivi bs={BS} bits={bits} build", flush=True)
        tla.kivi_build_pages(desc, kd, vd, btd, dev(start), ptd, pages, int(start.max()))
        torch.cuda.synchronize()
        kc.lens = start.copy()
        want_pages = kc.oracle_pages()
        used = [p for p in _used_pages(kc, start) if p >= 0]
        assert np.array_equal(pages.cpu().numpy()[used], want_pages[used])
        rng = np.random.default_rng(BS + bits)
        max_ctx = int(start.max()) + steps
        ws = torch.empty(max(16, tla.kivi_workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
        lens = start.copy()
        k_host, v_host = kc.k.copy(), kc.v.copy()
        print(f"case kivi bs={BS} bits={bits} steps", flush=True)
        for step in range(steps):
            lens = lens + 1
            pos = lens - 1
            ent = kc.tables[np.arange(kc.S), pos // BS]
            slots = np.where(ent >= 0, ent * BS + pos % BS, -1).astype(np.int32)
            knew = inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16)
            vnew = inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16)
            out = torch.full_like(qd, float("nan"))
            tla.kivi_decode_step(desc, out, qd, dev(knew, orc.F16), dev(vnew, orc.F16), dev(slots), pages, ptd,
                                 kd, vd, btd, dev(lens), max_ctx, ws)
            torch.cuda.synchronize()
            orc.reshape_and_cache(knew, vnew, k_host, v_host, slots)
            kc.k, kc.v, kc.lens = k_host, v_host, lens
            want_pages = kc.oracle_pages()
            assert_close(out, _kivi_ref(kc, want_pages), orc.F16, ATOL_KIVI, f"bs={BS} bits={bits} step {step}")
        assert np.array_equal(host_bits(kd), k_host) and np.array_equal(host_bits(vd), v_host)
        used = [p for p in _used_pages(kc, lens) if p >= 0]
        assert np.array_equal(pages.cpu().numpy()[used], want_pages[used])
        for pp in (-1, 2):
            print(f"case kivi bs={BS} bits={bits} decode pp={pp}", flush=True)
            assert_close(_run_decode(kc, want_pages, pp), _kivi_ref(kc, want_pages), orc.F16, ATOL_KIVI,
                         f"bs={BS} bits={bits} pp={pp}")


# ---------------------------------------------------------------------------
# build-ahead: pages written in eighths over the steps before they complete
# ---------------------------------------------------------------------------

# (L0 - R) mod 32 of the starting lengths: the next page's first eighth due
# one step ago (31, 24: the prefix build writes the page whole), at the first
# step (23), in mid window (27: five eighths due), later (16, 0)
_AHEAD_PHASES = [31, 24, 23, 27, 16, 0]


def _signed_zero_page(kc, s, L0):
    """Sequence s's next page to be quantised: every present token gets
    zeros of random sign in K channels 0-7 (octet 0) and V channels 32-63
    (group 1), so that each of those groups' min and max is a tie whose sign
    only the sequential scan order fixes."""
    P = orc.kivi_quantized_len(int(L0), kc.R) // 32
    rng = np.random.default_rng(1000 + s)
    for t in range(32 * P, min(32 * P + 32, int(L0))):
        blk = kc.tables[s, t // kc.BS]
        if blk < 0:
            continue
        for h in range(kc.n_kv):
            kc.k[blk, h, 0:8, t % kc.BS] = rng.choice([0x0000, 0x8000], 8)
            kc.v[blk, h, 32:64, t % kc.BS] = rng.choice([0x0000, 0x8000], 32)


@pytest.mark.parametrize("mode,bits,BS,R", [
    ("step", 4, 16, 128), ("step", 8, 16, 128), ("step", 4, 8, 9), ("step", 8, 64, 40), ("step", 4, 256, 128),
    ("append", 4, 16, 128), ("append", 8, 32, 9), ("alternate", 4, 16, 40), ("step", 4, 16, 8),
])
def test_build_ahead_pages_bit_exact_at_every_step(mode, bits, BS, R):
    """desc.build_ahead = 1 against the oracle, which quantises each page
    whole when the length completes it.  The starting lengths put every
    sequence at a different phase of its next page's eighths (the prefix
    build writes that page whole when its first eighth is already due); then
    40 appends through the fused step ('step'), through tl_kivi_append and
    the decode ('append'), or the two in turn ('alternate').  After every
    step the pages of every sequence are the oracle's bit for bit and the
    output matches the oracle.  With R = 8 the setting builds on completion.
    Signed zeros fill some groups of each sequence's next page; a window
    block of sequence 2 is a hole."""
    steps = 40
    start = np.array([R + 32 * k + o for k, o in zip([4, 2, 7, 0, 3, 1], _AHEAD_PHASES)], np.int32)
    kc = KiviCase(90 + BS + R + bits, start + steps, H=32, extra_blocks=1, bits=bits, BS=BS, R=R)
    for s, L0 in enumerate(start):
        _signed_zero_page(kc, s, L0)
    hole_lb = (int(start[2]) + 5) // BS
    kc.tables[2, hole_lb] = -1
    qd, kd, vd = dev(kc.q, orc.F16), dev(kc.k, orc.F16), dev(kc.v, orc.F16)
    btd, ptd = dev(kc.tables), dev(kc.page_tables)
    pages = torch.zeros(kc.num_pages, kc.n_kv, kc.page_bytes, dtype=torch.uint8, device="cuda")
    desc = tla.make_kivi_desc(qd, kd, btd, ptd, kc.num_pages, kc.n_kv, kc.scale, residual_length=R,
                              bits=bits, build_ahead=True)
    assert desc.build_ahead == 1 and desc.block_size == BS
    print(f"case build-ahead {mode} bits={bits} bs={BS} R={R}", flush=True)
    tla.kivi_build_pages(desc, kd, vd, btd, dev(start), ptd, pages, int(start.max()))
    rng = np.random.default_rng(BS * 7 + R + bits)
    max_ctx = int(start.max()) + steps
    ws = torch.empty(max(16, tla.kivi_workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
    lens = start.copy()
    k_host, v_host = kc.k.copy(), kc.v.copy()
    for step in range(steps):
        lens = lens + 1
        pos = lens - 1
        ent = kc.tables[np.arange(kc.S), pos // BS]
        slots = np.where(ent >= 0, ent * BS + pos % BS, -1).astype(np.int32)
        knew = inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16)
        vnew = inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16)
        out = torch.full_like(qd, float("nan"))
        fused = mode == "step" or (mode == "alternate" and step % 2 == 0)
        if fused:
            tla.kivi_decode_step(desc, out, qd, dev(knew, orc.F16), dev(vnew, orc.F16), dev(slots), pages, ptd,
                                 kd, vd, btd, dev(lens), max_ctx, ws)
        else:
            tla.kivi_append(desc, dev(knew, orc.F16), dev(vnew, orc.F16), kd, vd, dev(slots), btd, dev(lens),
                            ptd, pages)
            tla.kivi_paged_attention_decode(desc, out, qd, pages, ptd, kd, vd, btd, dev(lens), max_ctx, ws)
        torch.cuda.synchronize()
        orc.reshape_and_cache(knew, vnew, k_host, v_host, slots)
        kc.k, kc.v, kc.lens = k_host, v_host, lens
        want_pages = kc.oracle_pages()
        used = [p for p in _used_pages(kc, lens) if p >= 0]
        assert np.array_equal(pages.cpu().numpy()[used], want_pages[used]), f"pages after step {step}"
        assert_close(out, _kivi_ref(kc, want_pages), orc.F16, ATOL_KIVI, f"{mode} step {step}")
    assert np.array_equal(host_bits(kd), k_host) and np.array_equal(host_bits(vd), v_host)


@pytest.mark.parametrize("style,bits", [(tla.ROPE_HALVES, 4), (tla.ROPE_ADJACENT, 8)])
def test_build_ahead_pre_rope_step(style, bits):
    """build_ahead with the keys held before RoPE (tl_kivi_decode_step_pre_rope):
    the pages hold unrotated keys, bit for bit the oracle's at every step."""
    from test_oracle import rope_tables
    steps, R = 36, 128
    start = np.array([R + 32 * k + o for k, o in zip([4, 2, 7, 0, 3, 1], _AHEAD_PHASES)], np.int32)
    kc = KiviCase(77 + bits, start + steps, H=32, extra_blocks=1, bits=bits, R=R)
    cos_t, sin_t = rope_tables(1040, 128)
    qd, kd, vd = dev(kc.q, orc.F16), dev(kc.k, orc.F16), dev(kc.v, orc.F16)
    btd, ptd = dev(kc.tables), dev(kc.page_tables)
    pages = torch.zeros(kc.num_pages, kc.n_kv, kc.page_bytes, dtype=torch.uint8, device="cuda")
    desc = tla.make_kivi_desc(qd, kd, btd, ptd, kc.num_pages, kc.n_kv, kc.scale, residual_length=R,
                              bits=bits, pre_rope_keys=True, build_ahead=True)
    print(f"case build-ahead pre-rope style={style} bits={bits}", flush=True)
    tla.kivi_build_pages(desc, kd, vd, btd, dev(start), ptd, pages, int(start.max()))
    rng = np.random.default_rng(33 + bits)
    max_ctx = int(start.max()) + steps
    ws = torch.empty(max(16, tla.kivi_workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
    cos_d, sin_d = dev(cos_t), dev(sin_t)
    lens = start.copy()
    k_host, v_host = kc.k.copy(), kc.v.copy()
    for step in range(steps):
        lens = lens + 1
        pos = (lens - 1).astype(np.int32)
        slots = (kc.tables[np.arange(kc.S), pos // 16] * 16 + pos % 16).astype(np.int32)
        knew = inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16)
        vnew = inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16)
        out = torch.full_like(qd, float("nan"))
        tla.kivi_decode_step_pre_rope(desc, out, qd, dev(knew, orc.F16), dev(vnew, orc.F16), dev(slots), pages,
                                      ptd, kd, vd, btd, dev(lens), max_ctx, cos_d, sin_d, style, ws)
        torch.cuda.synchronize()
        orc.reshape_and_cache(knew, vnew, k_host, v_host, slots)
        kc.k, kc.v, kc.lens = k_host, v_host, lens
        want_pages = kc.oracle_pages()
        used = [p for p in _used_pages(kc, lens) if p >= 0]
        assert np.array_equal(pages.cpu().numpy()[used], want_pages[used]), f"pages after step {step}"
        want = orc.kivi_paged_attention(kc.q, orc.F16, want_pages, kc.page_tables, kc.k, kc.v, kc.tables, kc.lens,
                                        kc.n_kv, kc.R, kc.scale, orc.GROUPED, bits, pre_rope=(cos_t, sin_t, style))
        assert_close(out, want, orc.F16, ATOL_KIVI, f"step {step}")


def test_build_ahead_full_batch_mixed_lengths():
    """The benchmark's mixed-length workload (batch 64, sequence s at
    4096 + s mod 32 tokens, R = 128) with build_ahead, over 40 fused steps:
    at each step a quarter of the sequences write an eighth of a page and
    two complete one.  Pages of every sequence bit for bit at the end;
    outputs of 16 sequences against the oracle at the last step."""
    steps = 40
    start = np.array([4096 + s % 32 for s in range(64)], np.int32)
    kc = KiviCase(82, start + steps, H=32, extra_blocks=1)
    qd, kd, vd = dev(kc.q, orc.F16), dev(kc.k, orc.F16), dev(kc.v, orc.F16)
    btd, ptd = dev(kc.tables), dev(kc.page_tables)
    pages = torch.zeros(kc.num_pages, kc.n_kv, kc.page_bytes, dtype=torch.uint8, device="cuda")
    desc = tla.make_kivi_desc(qd, kd, btd, ptd, kc.num_pages, kc.n_kv, kc.scale, residual_length=kc.R,
                              build_ahead=True)
    tla.kivi_build_pages(desc, kd, vd, btd, dev(start), ptd, pages, int(start.max()))
    rng = np.random.default_rng(16)
    max_ctx = int(start.max()) + steps
    ws = torch.empty(max(16, tla.kivi_workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
    lens = start.copy()
    print("case build-ahead full batch, mixed lengths", flush=True)
    for step in range(steps):
        lens = lens + 1
        pos = lens - 1
        slots = (kc.tables[np.arange(kc.S), pos // 16] * 16 + pos % 16).astype(np.int32)
        knew = inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16)
        vnew = inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16)
        out = torch.full_like(qd, float("nan"))
        tla.kivi_decode_step(desc, out, qd, dev(knew, orc.F16), dev(vnew, orc.F16), dev(slots), pages, ptd, kd, vd,
                             btd, dev(lens), max_ctx, ws)
        orc.reshape_and_cache(knew, vnew, kc.k, kc.v, slots)
    torch.cuda.synchronize()
    kc.lens = lens
    want_pages = kc.oracle_pages()
    used = [p for p in _used_pages(kc, lens) if p >= 0]
    assert np.array_equal(pages.cpu().numpy()[used], want_pages[used])
    assert np.array_equal(host_bits(kd), kc.k) and np.array_equal(host_bits(vd), kc.v)
    sub = np.array([0, 1, 5, 9, 15, 16, 22, 23, 24, 31, 40, 47, 50, 55, 56, 63])
    want = orc.kivi_paged_attention(np.ascontiguousarray(kc.q[sub]), orc.F16, want_pages,
                                    np.ascontiguousarray(kc.page_tables[sub]), kc.k, kc.v,
                                    np.ascontiguousarray(kc.tables[sub]), np.ascontiguousarray(lens[sub]),
                                    kc.n_kv, kc.R, kc.scale, orc.GROUPED, kc.bits)
    assert_close(out[torch.from_numpy(sub).cuda()], want, orc.F16, ATOL_KIVI, "full batch")


@pytest.mark.parametrize("H,n_kv,pp", [(32, 1, 0), (32, 1, 4), (64, 8, 4), (48, 2, -1)])
def test_build_ahead_head_slices_and_split_k(H, n_kv, pp):
    """build_ahead with GQA groups wider than one wavefront's 16 heads (two
    or more workgroups per (sequence, kv head), of which one writes the
    piece) and with split-K plans (the piece written by the last
    partition's workgroup): pages bit for bit and outputs against the
    oracle after each of 36 fused steps."""
    steps, R = 36, 128
    start = np.array([R + 32 * k + o for k, o in zip([4, 2, 7, 0, 3, 1], _AHEAD_PHASES)], np.int32)
    kc = KiviCase(95 + H + n_kv + pp, start + steps, H=H, n_kv=n_kv, extra_blocks=1, R=R)
    qd, kd, vd = dev(kc.q, orc.F16), dev(kc.k, orc.F16), dev(kc.v, orc.F16)
    btd, ptd = dev(kc.tables), dev(kc.page_tables)
    pages = torch.zeros(kc.num_pages, kc.n_kv, kc.page_bytes, dtype=torch.uint8, device="cuda")
    desc = tla.make_kivi_desc(qd, kd, btd, ptd, kc.num_pages, kc.n_kv, kc.scale, residual_length=R,
                              partition_pages=pp, build_ahead=True)
    print(f"case build-ahead H={H} n_kv={n_kv} pp={pp}", flush=True)
    tla.kivi_build_pages(desc, kd, vd, btd, dev(start), ptd, pages, int(start.max()))
    rng = np.random.default_rng(H * 3 + n_kv + pp)
    max_ctx = int(start.max()) + steps
    ws = torch.empty(max(16, tla.kivi_workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
    lens = start.copy()
    k_host, v_host = kc.k.copy(), kc.v.copy()
    for step in range(steps):
        lens = lens + 1
        pos = lens - 1
        slots = (kc.tables[np.arange(kc.S), pos // 16] * 16 + pos % 16).astype(np.int32)
        knew = inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16)
        vnew = inputs.encode(rng.standard_normal((kc.S, kc.n_kv, 128), dtype=np.float32), orc.F16)
        out = torch.full_like(qd, float("nan"))
        tla.kivi_decode_step(desc, out, qd, dev(knew, orc.F16), dev(vnew, orc.F16), dev(slots), pages, ptd,
                             kd, vd, btd, dev(lens), max_ctx, ws)
        torch.cuda.synchronize()
        orc.reshape_and_cache(knew, vnew, k_host, v_host, slots)
        kc.k, kc.v, kc.lens = k_host, v_host, lens
        want_pages = kc.oracle_pages()
        used = [p for p in _used_pages(kc, lens) if p >= 0]
        assert np.array_equal(pages.cpu().numpy()[used], want_pages[used]), f"pages after step {step}"
        assert_close(out, _kivi_ref(kc, want_pages), orc.F16, ATOL_KIVI, f"H={H} n_kv={n_kv} pp={pp} step {step}")


def test_build_ahead_step_graph_replay_matches_eager():
    """The fused step with build_ahead captured in a HIP graph: 40 replays
    (each its own step, lengths and slots advanced through device buffers)
    give the eager run's pages and outputs bit for bit."""
    steps, R = 40, 128
    start = np.array([R + 32 * k + o for k, o in zip([4, 2, 7, 0, 3, 1], _AHEAD_PHASES)], np.int32)
    rng = np.random.default_rng(71)
    knew = [inputs.encode(rng.standard_normal((6, 8, 128), dtype=np.float32), orc.F16) for _ in range(steps)]
    vnew = [inputs.encode(rng.standard_normal((6, 8, 128), dtype=np.float32), orc.F16) for _ in range(steps)]
    results = []
    for graphed in (False, True):
        kc = KiviCase(97, start + steps, H=32, extra_blocks=1, R=R)
        qd, kd, vd = dev(kc.q, orc.F16), dev(kc.k, orc.F16), dev(kc.v, orc.F16)
        btd, ptd = dev(kc.tables), dev(kc.page_tables)
        pages = torch.zeros(kc.num_pages, kc.n_kv, kc.page_bytes, dtype=torch.uint8, device="cuda")
        desc = tla.make_kivi_desc(qd, kd, btd, ptd, kc.num_pages, kc.n_kv, kc.scale, residual_length=R,
                                  build_ahead=True)
        tla.kivi_build_pages(desc, kd, vd, btd, dev(start), ptd, pages, int(start.max()))
        max_ctx = int(start.max()) + steps
        ws = torch.empty(max(16, tla.kivi_workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
        sl = dev(start)
        slot_d = torch.zeros(kc.S, dtype=torch.int32, device="cuda")
        kn = torch.zeros(kc.S, kc.n_kv, 128, dtype=torch.float16, device="cuda")
        vn = torch.zeros_like(kn)
        out = torch.zeros_like(qd)
        outs = []
        stream = torch.cuda.Stream()
        graph = None
        print(f"case build-ahead graph={graphed}", flush=True)
        for step in range(steps):
            lens = start + step + 1
            pos = lens - 1
            sl.copy_(dev(lens))
            slot_d.copy_(dev((kc.tables[np.arange(kc.S), pos // 16] * 16 + pos % 16).astype(np.int32)))
            kn.copy_(dev(knew[step], orc.F16))
            vn.copy_(dev(vnew[step], orc.F16))
            torch.cuda.synchronize()
            if graphed:
                if graph is None:
                    graph = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(graph, stream=stream):
                        tla.kivi_decode_step(desc, out, qd, kn, vn, slot_d, pages, ptd, kd, vd, btd, sl, max_ctx, ws,
                                             torch.cuda.current_stream())
                graph.replay()
            else:
                tla.kivi_decode_step(desc, out, qd, kn, vn, slot_d, pages, ptd, kd, vd, btd, sl, max_ctx, ws)
            torch.cuda.synchronize()
            outs.append(out.clone())
        results.append((outs, pages.clone(), kd.clone(), vd.clone()))
    (o0, p0, k0, v0), (o1, p1, k1, v1) = results
    assert torch.equal(p0, p1) and torch.equal(k0, k1) and torch.equal(v0, v1)
    for step in range(steps):
        assert torch.equal(o0[step], o1[step]), f"step {step}"
