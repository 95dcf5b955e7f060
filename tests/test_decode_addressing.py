"""Host-side check of the matrix-core decode's load addresses.

The wavefronts of tl_mfma_wave.hpp (fp8_wave, mfma2_wave) compute every
lane's K and V load addresses from (block size, lane, iteration).  This test
restates that address arithmetic on the CPU for every lane and iteration of
small batches (ragged lengths, table holes, entries past the pool) and
checks two things against the pool layout [N][n_kv][D][BS] (cache_kernels.cu
:74-83, an independent definition of where token t, dim d lives):
  - bounds: every load of every lane, prefetches included, lies inside the
    pool (holes and tokens past the partition load block 0);
  - mapping: for a token of a valid block, the address a lane loads is the
    element the MFMA slot it feeds expects (K: dims 4 j + kg of token pair /
    quad m; V: dims 16 dt + m of the lane's 8- or 16-token run).
It covers the ways the kernels split work: 1, 2 and 4 wavefronts striding
over a partition, runs of 1, 2 and 4 whole partitions per wavefront, and
single pass."""
import numpy as np
import pytest

D = 128


def table_entry(table, tok, t1, max_blocks, num_blocks, BS):
    """table_blocks: physical block of token tok, -1 for a hole, a token at
    or past t1, a row entry past max_blocks or an id past the pool.  The
    kernel reads the row entry at the index clamped to the row whatever the
    token, so that read must stay inside the row."""
    lb = tok // BS
    idx = min(lb, max_blocks - 1)
    assert 0 <= idx < max_blocks and idx < table.shape[0]
    e = int(table[idx])
    if tok >= t1 or lb >= max_blocks:
        return -1
    return -1 if e >= num_blocks else e


def wave_loads(E, BS, table, t0, t1, first_it, step, max_blocks, num_blocks, n_kv, kvh):
    """Yields (it, kind, j, addr, width) for every load of one wavefront
    (addr: the 64 lanes' byte offsets into the pool), restating the kernel's
    address formulas."""
    TPI = 32 if E == 2 else 64
    RB = E * BS
    block_bytes = D * RB
    pool_stride = n_kv * block_bytes
    NB = 1 if BS >= TPI else TPI // BS
    lanes = np.arange(64)
    m, kg = lanes & 15, lanes >> 4
    unit_k = 2 if E == 2 else 4          # tokens per K lane-group row: pairs (2-byte) or quads (FP8)
    run = 8 if E == 2 else 16            # tokens of one V run
    kb = (unit_k * m) // BS if NB > 1 else np.zeros(64, int)
    vb = (run * kg) // BS if NB > 1 else np.zeros(64, int)
    kmod = BS if NB > 1 else TPI
    kbase0 = kvh * block_bytes + RB * kg + E * ((unit_k * m) % kmod)
    vbase0 = kvh * block_bytes + RB * m + E * ((run * kg) % kmod)

    def blocks(it):
        return [table_entry(table, it + BS * i, t1, max_blocks, num_blocks, BS) for i in range(NB)]

    def ib(it):
        return E * (it % BS) if BS > TPI else 0

    def loads(it, cur):
        kblk = np.array([max(cur[b], 0) for b in kb])
        vblk = np.array([max(cur[b], 0) for b in vb])
        for j in range(32):
            addr = kbase0 + ib(it) + kblk * pool_stride + 4 * RB * j
            yield "k", j, addr, 4
        for dt in range(8):
            addr = vbase0 + ib(it) + vblk * pool_stride + 16 * RB * dt
            yield "v", dt, addr, 16

    # the first iteration's loads and, in every iteration, the next one's
    # are issued unconditionally (a missing iteration reads block 0)
    it = first_it
    yield from ((it, k, j, a, w) for k, j, a, w in loads(it, blocks(it)))
    while it < t1:
        yield from ((it + step, k, j, a, w) for k, j, a, w in loads(it + step, blocks(it + step)))
        it += step


def element(E, BS, n_kv, ph, kvh, d, tok):
    """Pool layout [N][n_kv][D][BS] with E-byte elements."""
    return ((ph * n_kv + kvh) * D + d) * BS * E + (tok % BS) * E


def check_wave(E, BS, table, L, t0, t1, first_it, step, max_blocks, num_blocks, n_kv, kvh):
    pool_bytes = num_blocks * n_kv * D * BS * E
    TPI = 32 if E == 2 else 64
    lanes = np.arange(64)
    m, kg = lanes & 15, lanes >> 4
    n = 0
    for it, kind, j, addr, width in wave_loads(E, BS, table, t0, t1, first_it, step, max_blocks, num_blocks,
                                               n_kv, kvh):
        assert (addr >= 0).all() and (addr + width <= pool_bytes).all(), (kind, it, j)
        # mapping: the first element of each lane's load, for a valid token
        if kind == "k":
            tok = it + (2 * m if E == 2 else 4 * m)
            d = 4 * j + kg
        else:
            tok = it + (8 * kg if E == 2 else 16 * kg)
            d = 16 * j + m
        lb = tok // BS
        ph = np.where((tok < t1) & (lb < max_blocks), table[np.minimum(lb, max_blocks - 1)], -1)
        ph = np.where(ph >= num_blocks, -1, ph)
        ok = ph >= 0
        want = element(E, BS, n_kv, ph, kvh, d, tok)
        assert (addr[ok] == want[ok]).all(), (kind, it, j)
        n += 1
    return n


def make_tables(rng, lens, BS, holes, past_pool):
    nbs = [(L + BS - 1) // BS for L in lens]
    N = sum(nbs) + 3
    perm = rng.permutation(N)
    mb = max(max(nbs), 1)
    table = np.full((len(lens), mb), -1, np.int64)
    off = 0
    for s, nb in enumerate(nbs):
        table[s, :nb] = perm[off:off + nb]
        off += nb
    for _ in range(holes):
        s = int(rng.integers(len(lens)))
        if nbs[s]:
            table[s, int(rng.integers(nbs[s]))] = -1
    for _ in range(past_pool):
        s = int(rng.integers(len(lens)))
        if nbs[s]:
            table[s, int(rng.integers(nbs[s]))] = N + 5
    return table, N, mb


@pytest.mark.parametrize("E,BS", [(2, 8), (2, 16), (2, 32), (2, 64), (2, 128), (2, 256),
                                  (1, 16), (1, 32), (1, 64), (1, 128), (1, 256)])
def test_matrix_core_decode_loads_stay_in_the_pool_and_hit_their_elements(E, BS):
    rng = np.random.default_rng(E * 1000 + BS)
    lens = [1, 31, 33, 64, 65, 511, 513, 1100, 2049]
    n_kv = 2
    table, N, mb = make_tables(rng, lens, BS, holes=3, past_pool=2)
    TPI = 32 if E == 2 else 64
    checked = 0
    for s, L in enumerate(lens):
        kvh = s % n_kv
        # single pass, 4 wavefronts
        for w in range(4):
            checked += check_wave(E, BS, table[s], L, 0, L, w * TPI, 4 * TPI, mb, N, n_kv, kvh)
        for PT in (512, 1024):
            for part in range((L + PT - 1) // PT):
                t0, t1 = part * PT, min(part * PT + PT, L)
                for NW in (1, 2, 4):              # wavefronts striding over one partition
                    for w in range(NW):
                        checked += check_wave(E, BS, table[s], L, t0, t1, t0 + w * TPI, NW * TPI, mb, N, n_kv,
                                              kvh)
                # whole partitions per wavefront: runs of 1, 2 and 4 partitions
                for k in (1, 2, 4):
                    if part % k == 0:
                        checked += check_wave(E, BS, table[s], L, t0, min(t0 + k * PT, L), t0, TPI, mb, N, n_kv,
                                              kvh)
    assert checked > 100


def test_partial_slots_stay_in_the_workspace():
    """write_partial: slot (seq * H + head) * P + part and dims 16 dt + 4 kg
    + 0..3 of a 128-dim row; the wave-per-partition grid's partitions
    4 pg + w that reach P return before writing."""
    S, H, n_kv, P = 3, 32, 8, 7
    group = H // n_kv
    groups = (P + 3) // 4
    slots = set()
    for pg in range(groups):
        for w in range(4):
            part = 4 * pg + w
            if part >= P:
                continue
            for seq in range(S):
                for kvh in range(n_kv):
                    for gi in range(group):
                        head = kvh * group + gi
                        pi = (seq * H + head) * P + part
                        assert 0 <= pi < S * H * P
                        slots.add(pi)
    assert len(slots) == S * H * P
    dims = {16 * dt + 4 * kg + r for dt in range(8) for kg in range(4) for r in range(4)}
    assert dims == set(range(128))
