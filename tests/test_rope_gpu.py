"""RoPE + reshape_and_cache on the GPU, bit-exact against the oracle."""
import numpy as np
import pytest
import torch

import inputs
import oracle_lib as orc
import tl_attn as tla
from gpu_util import dev, host_bits
from test_oracle import rope_tables

pytestmark = pytest.mark.gpu


def _case(seed, T, H, n_kv, D, BS, N, code, max_pos):
    rng = np.random.default_rng(seed)
    q = inputs.encode(rng.standard_normal((T, H, D), dtype=np.float32), code)
    key = inputs.encode(rng.standard_normal((T, n_kv, D), dtype=np.float32), code)
    val = inputs.encode(rng.standard_normal((T, n_kv, D), dtype=np.float32), code)
    slots = rng.choice(N * BS, size=T, replace=False).astype(np.int32)
    slots[::7] = -1
    pos = rng.integers(0, max_pos, size=T).astype(np.int32)
    pos[3 % T] = max_pos + 5                             # past the tables: nothing written
    kc = inputs.encode(rng.standard_normal((N, n_kv, D, BS), dtype=np.float32), code)
    vc = inputs.encode(rng.standard_normal((N, n_kv, D, BS), dtype=np.float32), code)
    return q, key, val, slots, pos, kc, vc


@pytest.mark.parametrize("style", [tla.ROPE_ADJACENT, tla.ROPE_HALVES])
@pytest.mark.parametrize("code", [orc.F16, orc.BF16, orc.F32])
@pytest.mark.parametrize("T,H,n_kv,D,BS", [(64, 32, 8, 128, 16), (37, 8, 2, 64, 32), (5, 4, 4, 256, 16)])
def test_rope_reshape_and_cache_bit_exact(style, code, T, H, n_kv, D, BS):
    N, max_pos = 48, 4096
    q, key, val, slots, pos, kc, vc = _case(T + D + style, T, H, n_kv, D, BS, N, code, max_pos)
    cos_t, sin_t = rope_tables(max_pos, D)
    qd, kd, vd = dev(q, code), dev(key, code), dev(val, code)
    kcd, vcd = dev(kc, code), dev(vc, code)
    q_out = torch.zeros_like(qd)
    print(f"case rope style={style} code={code} T={T} D={D}", flush=True)
    tla.rope_reshape_and_cache(qd, kd, vd, kcd, vcd, dev(slots), dev(pos), dev(cos_t), dev(sin_t), style,
                               q_out=q_out)
    torch.cuda.synchronize()
    q_ref = np.zeros_like(q)
    orc.rope_reshape_and_cache(q, q_ref, key, val, kc, vc, slots, pos, cos_t, sin_t, code, style)
    assert np.array_equal(host_bits(q_out), q_ref)
    assert np.array_equal(host_bits(kcd), kc)
    assert np.array_equal(host_bits(vcd), vc)


@pytest.mark.parametrize("style", [tla.ROPE_ADJACENT, tla.ROPE_HALVES])
@pytest.mark.parametrize("code", [orc.F16, orc.BF16, orc.F32])
@pytest.mark.parametrize("T,H,n_kv,D,BS", [(64, 32, 8, 128, 16), (33, 8, 2, 64, 32), (300, 4, 2, 128, 16)])
def test_rope_decode_append_bit_exact(style, code, T, H, n_kv, D, BS):
    """One token per block (a decode step: whole block rows for up to 256
    tokens, element stores past that) over a pool of random bytes; token 7
    shares token 3's block, token 9 shares token 5's block but its position
    is past the tables (so token 5 still owns the block), token 11 is
    padded."""
    N, max_pos = 2 * T + 8, 4096
    q, key, val, _, pos, kc, vc = _case(T * 3 + D + style, T, H, n_kv, D, BS, N, code, max_pos)
    rng = np.random.default_rng(T + style)
    slots = (rng.permutation(N)[:T] * BS + rng.integers(0, BS, size=T)).astype(np.int32)
    slots[7] = slots[3] - slots[3] % BS + (slots[3] % BS + 1) % BS
    slots[9] = slots[5] - slots[5] % BS + (slots[5] % BS + 1) % BS
    pos[9] = max_pos + 1
    slots[11] = -1
    cos_t, sin_t = rope_tables(max_pos, D)
    qd, kd, vd = dev(q, code), dev(key, code), dev(val, code)
    kcd, vcd = dev(kc, code), dev(vc, code)
    q_out = torch.zeros_like(qd)
    print(f"case rope append style={style} code={code} T={T} D={D} BS={BS}", flush=True)
    tla.rope_reshape_and_cache(qd, kd, vd, kcd, vcd, dev(slots), dev(pos), dev(cos_t), dev(sin_t), style,
                               q_out=q_out)
    torch.cuda.synchronize()
    q_ref = np.zeros_like(q)
    orc.rope_reshape_and_cache(q, q_ref, key, val, kc, vc, slots, pos, cos_t, sin_t, code, style)
    assert np.array_equal(host_bits(q_out), q_ref)
    assert np.array_equal(host_bits(kcd), kc)
    assert np.array_equal(host_bits(vcd), vc)


def test_rope_in_place_equals_out_of_place_and_graph_replay():
    code, style = orc.BF16, tla.ROPE_ADJACENT
    T, H, n_kv, D, BS, N, max_pos = 64, 32, 8, 128, 16, 64, 8192
    q, key, val, slots, pos, kc, vc = _case(77, T, H, n_kv, D, BS, N, code, max_pos)
    cos_t, sin_t = dev(rope_tables(max_pos, D)[0]), dev(rope_tables(max_pos, D)[1])
    qd, kd, vd, sd, pd = dev(q, code), dev(key, code), dev(val, code), dev(slots), dev(pos)
    kc0, vc0 = dev(kc, code), dev(vc, code)
    a_out = torch.zeros_like(qd)
    ka, va = kc0.clone(), vc0.clone()
    print("case rope in place", flush=True)
    tla.rope_reshape_and_cache(qd, kd, vd, ka, va, sd, pd, cos_t, sin_t, style, q_out=a_out)
    qi = qd.clone()
    kb, vb = kc0.clone(), vc0.clone()
    tla.rope_reshape_and_cache(qi, kd, vd, kb, vb, sd, pd, cos_t, sin_t, style)
    torch.cuda.synchronize()
    keep = torch.from_numpy((pos < max_pos)).cuda()
    assert torch.equal(qi[keep].view(torch.int16), a_out[keep].view(torch.int16))
    assert torch.equal(ka.view(torch.int16), kb.view(torch.int16))
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    g_out = torch.zeros_like(qd)
    kg, vg = kc0.clone(), vc0.clone()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=cap):
        tla.rope_reshape_and_cache(qd, kd, vd, kg, vg, sd, pd, cos_t, sin_t, style, q_out=g_out, stream=cap)
    for _ in range(3):
        g_out.zero_()
        kg.copy_(kc0)
        vg.copy_(vc0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(g_out.view(torch.int16), a_out.view(torch.int16))
        assert torch.equal(kg.view(torch.int16), ka.view(torch.int16))
        assert torch.equal(vg.view(torch.int16), va.view(torch.int16))
