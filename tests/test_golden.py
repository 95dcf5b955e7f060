"""The committed golden fixtures (tests/golden/, written by
tests/golden/make_golden.py with the oracle).

CPU: the seeded inputs still regenerate to the recorded digests, and the
oracle still reproduces every fixture (codec bytes exactly, attention to
fp32 rounding of the stored values), so a change to the generator or the
oracle cannot pass unnoticed.
GPU: the HIP kernels against the fixtures themselves, not the live oracle:
codec bytes bit-exact; attention within max-abs 2e-3 (fp16 / bf16 KV) or
1e-2 (INT4 / FP8 KV) plus half an output ulp."""
import numpy as np
import pytest

import golden_cases as gc
import oracle_lib as orc


def _close(a, b, tol=2e-6):
    np.testing.assert_allclose(a, b, rtol=0, atol=tol)


def test_golden_c1_inputs_and_oracle():
    g = gc.load("c1_fp16_batch4")
    c = gc.c1_fp16_batch4()
    assert gc.digest(c.q, c.k_cache, c.v_cache, c.tables, c.seq_lens) == str(g["digest"])
    assert np.array_equal(c.seq_lens, g["lens"])
    for label, gqa in (("grouped", orc.GROUPED), ("modulo", orc.MODULO)):
        out = orc.paged_attention(c.q, orc.F16, c.k_cache, c.v_cache, orc.F16, c.tables, c.seq_lens, 8, c.scale,
                                  gqa)
        _close(out, g["out_" + label])


def test_golden_c2_inputs_and_oracle():
    g = gc.load("c2_bf16_varlen")
    c = gc.c2_bf16_varlen()
    assert gc.digest(c.q, c.k_cache, c.v_cache, c.tables, c.seq_lens) == str(g["digest"])
    out = orc.paged_attention(c.q, orc.BF16, c.k_cache, c.v_cache, orc.BF16, c.tables, c.seq_lens, 8, c.scale,
                              orc.GROUPED)
    _close(out, g["out"])


def test_golden_c3_kivi_inputs_pages_and_oracle():
    g = gc.load("c3_kivi_int4")
    kv = gc.KiviInputs()
    assert kv.digest() == str(g["digest"])
    pages = kv.pages()
    assert gc.digest(pages) == str(g["pages_digest"])
    out = orc.kivi_paged_attention(kv.q, orc.F16, pages, kv.page_tables, kv.k, kv.v, kv.tables, kv.lens, 8, kv.R,
                                   kv.scale, orc.GROUPED)
    _close(out, g["out"])


def test_golden_c4_fp8_inputs_and_oracle():
    g = gc.load("c4_fp8_e4m3")
    f8 = gc.Fp8Inputs()
    assert f8.digest() == str(g["digest"])
    assert np.float32(f8.ks) == g["k_scale"] and np.float32(f8.vs) == g["v_scale"]
    out = orc.paged_attention(f8.q, orc.BF16, f8.k8, f8.v8, orc.FP8, f8.tables, f8.lens, 8, f8.scale, orc.GROUPED,
                              0, f8.ks, f8.vs)
    _close(out, g["out"])


def test_golden_c5_prefill_inputs_and_oracle():
    g = gc.load("c5_prefill")
    pf = gc.PrefillInputs()
    assert pf.digest() == str(g["digest"])
    assert np.array_equal(pf.rows, g["rows"])
    c = pf.case
    full = orc.chunked_prefill(pf.q, orc.BF16, pf.cu, c.k_cache, c.v_cache, orc.BF16, c.tables, pf.lens, 2,
                               c.scale, orc.GROUPED)
    _close(full[pf.rows], g["out_rows"])


def test_golden_fp8_encode_and_kivi_codec_bytes():
    g = gc.load("fp8_e4m3_every_f16")
    bits = np.arange(65536, dtype=np.uint16)
    for label, mul in (("scale_1", 1.0), ("scale_inv448", 1.0 / 448.0)):
        out = np.empty(65536, np.uint8)
        orc.lib.orc_convert(orc.ptr(bits), orc.F16, orc.ptr(out), orc.FP8, bits.size, mul)
        assert np.array_equal(out, g[label])
    k = gc.load("kivi_codec")
    for D, O, G in gc.KIVI_VEC_PARAMS:
        x = gc.kivi_vectors(D)
        assert np.array_equal(x, k[f"x_{D}_{O}_{G}"])
        rec = orc.kivi_compress(x, D, O, G)
        assert np.array_equal(rec, k[f"rec_{D}_{O}_{G}"])
        assert np.array_equal(orc.kivi_decompress(rec, x.shape[0], D, O, G), k[f"back_{D}_{O}_{G}"])
    kt, vt = gc.kivi_page_tokens()
    assert np.array_equal(kt, k["page_k"]) and np.array_equal(vt, k["page_v"])
    page = orc.kivi_page_quantize(kt, vt)
    assert np.array_equal(page, k["page"])
    kd, vd = orc.kivi_page_dequant(page)
    assert np.array_equal(kd, k["page_k_back"]) and np.array_equal(vd, k["page_v_back"])


# ---------------------------------------------------------------------------
# the HIP kernels against the fixtures
# ---------------------------------------------------------------------------

def _gpu():
    import torch

    import tl_attn as tla
    from gpu_util import assert_close, dev
    return torch, tla, assert_close, dev


@pytest.mark.gpu
def test_golden_gpu_decode_c1_c2():
    torch, tla, assert_close, dev = _gpu()
    for name, make, code, maps in (("c1_fp16_batch4", gc.c1_fp16_batch4, orc.F16,
                                    (("grouped", tla.GQA_GROUPED), ("modulo", tla.GQA_MODULO))),
                                   ("c2_bf16_varlen", gc.c2_bf16_varlen, orc.BF16, (("", tla.GQA_GROUPED),))):
        g = gc.load(name)
        c = make()
        q, k, v, bt, sl = dev(c.q, code), dev(c.k_cache, code), dev(c.v_cache, code), dev(c.tables), dev(c.seq_lens)
        max_ctx = int(c.seq_lens.max())
        for label, gqa in maps:
            for pt in (-1, 512, 0):
                desc = tla.make_decode_desc(q, k, bt, 8, c.scale, gqa_map=gqa, partition_tokens=pt)
                ws = torch.empty(max(16, tla.workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
                out = torch.full_like(q, float("nan"))
                print(f"case golden {name} {label} pt={pt}", flush=True)
                tla.paged_attention_decode(desc, out, q, k, v, bt, sl, max_ctx, ws)
                torch.cuda.synchronize()
                want = g["out_" + label] if label else g["out"]
                assert_close(out, want.astype(np.float64), code, 2e-3, f"{name} {label} pt={pt}")


@pytest.mark.gpu
def test_golden_gpu_kivi_c3():
    torch, tla, assert_close, dev = _gpu()
    g = gc.load("c3_kivi_int4")
    kv = gc.KiviInputs()
    qd, kd, vd = dev(kv.q, orc.F16), dev(kv.k, orc.F16), dev(kv.v, orc.F16)
    btd, sld, ptd = dev(kv.tables), dev(kv.lens), dev(kv.page_tables)
    pages = torch.zeros(kv.num_pages, 8, tla.KIVI_PAGE_BYTES, dtype=torch.uint8, device="cuda")
    desc = tla.make_kivi_desc(qd, kd, btd, ptd, kv.num_pages, 8, kv.scale, residual_length=kv.R)
    print("case golden c3 kivi", flush=True)
    tla.kivi_build_pages(desc, kd, vd, btd, sld, ptd, pages, int(kv.lens.max()))
    torch.cuda.synchronize()
    assert gc.digest(pages.cpu().numpy()) == str(g["pages_digest"])
    max_ctx = int(kv.lens.max())
    ws = torch.empty(max(16, tla.kivi_workspace_bytes(desc, max_ctx)), dtype=torch.uint8, device="cuda")
    out = torch.full_like(qd, float("nan"))
    tla.kivi_paged_attention_decode(desc, out, qd, pages, ptd, kd, vd, btd, sld, max_ctx, ws)
    torch.cuda.synchronize()
    assert_close(out, g["out"].astype(np.float64), orc.F16, 1e-2, "c3 kivi")


@pytest.mark.gpu
def test_golden_gpu_fp8_c4():
    torch, tla, assert_close, dev = _gpu()
    g = gc.load("c4_fp8_e4m3")
    f8 = gc.Fp8Inputs()
    qd = dev(f8.q, orc.BF16)
    kd, vd = torch.from_numpy(f8.k8).cuda(), torch.from_numpy(f8.v8).cuda()
    bt, sl = dev(f8.tables), dev(f8.lens)
    for pt in (512, 0, -1):
        desc = tla.make_decode_desc(qd, kd, bt, 8, f8.scale, kv_dtype=tla.FP8_E4M3, gqa_map=tla.GQA_GROUPED,
                                    partition_tokens=pt, k_scale=f8.ks, v_scale=f8.vs)
        ws = torch.empty(max(16, tla.workspace_bytes(desc, 8192)), dtype=torch.uint8, device="cuda")
        out = torch.full_like(qd, float("nan"))
        print(f"case golden c4 fp8 pt={pt}", flush=True)
        tla.paged_attention_decode(desc, out, qd, kd, vd, bt, sl, 8192, ws)
        torch.cuda.synchronize()
        assert_close(out, g["out"].astype(np.float64), orc.BF16, 1e-2, f"c4 fp8 pt={pt}")


@pytest.mark.gpu
def test_golden_gpu_prefill_c5():
    torch, tla, assert_close, dev = _gpu()
    g = gc.load("c5_prefill")
    pf = gc.PrefillInputs()
    c = pf.case
    q = dev(pf.q, orc.BF16)
    k, v = dev(c.k_cache, orc.BF16), dev(c.v_cache, orc.BF16)
    bt, sl, cu = dev(c.tables), dev(pf.lens), dev(pf.cu)
    out = torch.full_like(q, float("nan"))
    desc = tla.make_prefill_desc(q, k, bt, len(pf.lens), 2, c.scale, num_prefill_seqs=2)
    print("case golden c5 prefill", flush=True)
    tla.chunked_prefill(desc, out, q, cu, k, v, bt, sl, int(pf.q_lens.max()))
    torch.cuda.synchronize()
    assert_close(out[torch.from_numpy(pf.rows).cuda()], g["out_rows"].astype(np.float64), orc.BF16, 2e-3, "c5")


@pytest.mark.gpu
def test_golden_gpu_codecs():
    torch, tla, assert_close, dev = _gpu()
    g = gc.load("fp8_e4m3_every_f16")
    x = dev(np.arange(65536, dtype=np.uint16), orc.F16)
    for label, mul in (("scale_1", 1.0), ("scale_inv448", 1.0 / 448.0)):
        out = torch.zeros(65536, dtype=torch.uint8, device="cuda")
        print(f"case golden fp8 encode {label}", flush=True)
        tla.convert_fp8(out, x, mul)
        torch.cuda.synchronize()
        got, want = out.cpu().numpy(), g[label]
        nan = (want & 0x7F) == 0x7F
        assert np.array_equal(got[~nan], want[~nan]) and ((got[nan] & 0x7F) == 0x7F).all()
    k = gc.load("kivi_codec")
    for D, O, G in gc.KIVI_VEC_PARAMS:
        xs = k[f"x_{D}_{O}_{G}"]
        n = xs.shape[0]
        rec = torch.zeros(n * tla.kivi_compressed_bytes(D, O, G), dtype=torch.uint8, device="cuda")
        back = torch.zeros(n, D, dtype=torch.float16, device="cuda")
        print(f"case golden kivi vectors D={D} O={O} G={G}", flush=True)
        tla.kivi_compress(dev(xs, orc.F16), rec, n, D, O, G)
        tla.kivi_decompress(rec, back, n, D, O, G)
        torch.cuda.synchronize()
        assert np.array_equal(rec.cpu().numpy(), k[f"rec_{D}_{O}_{G}"])
        assert np.array_equal(back.view(torch.int16).cpu().numpy().view(np.uint16).ravel(), k[f"back_{D}_{O}_{G}"])
