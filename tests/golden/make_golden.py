"""Writes the golden fixtures of tests/golden/ with the CPU oracle.

    python tests/golden/make_golden.py

Attention fixtures hold the digest of the seeded inputs (tests/golden_cases.py
regenerates them) and the oracle's output in fp32; codec fixtures hold the
bytes.  Nothing of the reference is run or imported: the oracle is this
repository's C restatement (oracle/tl_oracle.c), pinned by tests/test_oracle.py."""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

import golden_cases as gc  # noqa: E402
import oracle_lib as orc  # noqa: E402


def save(name, **arrays):
    np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrays)
    print("wrote", name, {k: v.shape for k, v in arrays.items()})


def main():
    c = gc.c1_fp16_batch4()
    outs = {}
    for label, gqa in (("grouped", orc.GROUPED), ("modulo", orc.MODULO)):
        outs[label] = orc.paged_attention(c.q, orc.F16, c.k_cache, c.v_cache, orc.F16, c.tables, c.seq_lens, 8,
                                          c.scale, gqa).astype(np.float32)
    save("c1_fp16_batch4", digest=np.array(gc.digest(c.q, c.k_cache, c.v_cache, c.tables, c.seq_lens)),
         lens=c.seq_lens, out_grouped=outs["grouped"], out_modulo=outs["modulo"])

    c = gc.c2_bf16_varlen()
    out = orc.paged_attention(c.q, orc.BF16, c.k_cache, c.v_cache, orc.BF16, c.tables, c.seq_lens, 8, c.scale,
                              orc.GROUPED).astype(np.float32)
    save("c2_bf16_varlen", digest=np.array(gc.digest(c.q, c.k_cache, c.v_cache, c.tables, c.seq_lens)),
         lens=c.seq_lens, out=out)

    kv = gc.KiviInputs()
    pages = kv.pages()
    out = orc.kivi_paged_attention(kv.q, orc.F16, pages, kv.page_tables, kv.k, kv.v, kv.tables, kv.lens, 8, kv.R,
                                   kv.scale, orc.GROUPED).astype(np.float32)
    save("c3_kivi_int4", digest=np.array(kv.digest()), pages_digest=np.array(gc.digest(pages)), out=out)

    f8 = gc.Fp8Inputs()
    out = orc.paged_attention(f8.q, orc.BF16, f8.k8, f8.v8, orc.FP8, f8.tables, f8.lens, 8, f8.scale, orc.GROUPED,
                              0, f8.ks, f8.vs).astype(np.float32)
    save("c4_fp8_e4m3", digest=np.array(f8.digest()), k_scale=np.float32(f8.ks), v_scale=np.float32(f8.vs),
         out=out)

    pf = gc.PrefillInputs()
    c = pf.case
    full = orc.chunked_prefill(pf.q, orc.BF16, pf.cu, c.k_cache, c.v_cache, orc.BF16, c.tables, pf.lens, 2,
                               c.scale, orc.GROUPED)
    save("c5_prefill", digest=np.array(pf.digest()), rows=pf.rows, out_rows=full[pf.rows].astype(np.float32))

    bits = np.arange(65536, dtype=np.uint16)
    codes = {}
    for label, mul in (("scale_1", 1.0), ("scale_inv448", 1.0 / 448.0)):
        out = np.empty(65536, np.uint8)
        orc.lib.orc_convert(orc.ptr(bits), orc.F16, orc.ptr(out), orc.FP8, bits.size, mul)
        codes[label] = out
    save("fp8_e4m3_every_f16", **codes)

    vec = {}
    for D, O, G in gc.KIVI_VEC_PARAMS:
        x = gc.kivi_vectors(D)
        rec = orc.kivi_compress(x, D, O, G)
        vec[f"x_{D}_{O}_{G}"] = x
        vec[f"rec_{D}_{O}_{G}"] = rec
        vec[f"back_{D}_{O}_{G}"] = orc.kivi_decompress(rec, x.shape[0], D, O, G)
    kt, vt = gc.kivi_page_tokens()
    page = orc.kivi_page_quantize(kt, vt)
    kd, vd = orc.kivi_page_dequant(page)
    save("kivi_codec", **vec, page_k=kt, page_v=vt, page=page, page_k_back=kd, page_v_back=vd)


if __name__ == "__main__":
    main()
