"""bench.py on the CPU: its refusals, and the work counts its rates divide by
against closed forms."""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def _run(*argv):
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *argv], capture_output=True, text=True,
                       timeout=120, cwd=ROOT)
    return r.returncode, json.loads(r.stdout.strip().splitlines()[-1])


def test_more_than_one_gpu_is_refused():
    rc, line = _run("--gpus", "2")
    assert rc == 2 and "one GPU" in line["error"]


def test_block_size_only_for_the_plain_decode_lines():
    for argv in (("--only", "kivi", "--block-size", "32"), ("--block-size", "32"),
                 ("--only", "fp8", "--block-size", "8")):
        rc, line = _run(*argv)
        assert rc == 2 and "--block-size" in line["error"], argv


def test_headline_algorithmic_bytes():
    """Batch 64, ctx 4096, 8 kv heads, d 128, 2-byte KV, bs 16: K and V once
    (2^30 B), q and out (64 x 32 x 128 x 2 B each), 256 table entries per
    sequence and the lengths: 1 074 856 192 B."""
    assert bench.BS == 16
    kv = 64 * 4096 * 8 * 128 * 2 * 2
    assert kv == 1 << 30
    expect = kv + 2 * 64 * 32 * 128 * 2 + 64 * 256 * 4 + 64 * 4
    assert expect == 1074856192
    assert bench.algorithmic_bytes([4096] * 64, 2) == expect
    # one token more per sequence reaches one more block per sequence
    assert bench.algorithmic_bytes([4097] * 64, 2) - expect == 64 * (8 * 128 * 2 * 2 + 4)


def test_prefill_flops_closed_form():
    """Chunks of one causal prompt cover the whole prompt's triangle: per q
    head P (P + 1) / 2 (query, key) pairs for a P-token prompt, 4 d FLOPs
    each, whatever the chunk size."""
    P = bench.PF_PROMPT
    expect = 4 * bench.D * P * (P + 1) // 2 * bench.PF_H * bench.PF_SEQS
    assert bench.prefill_flops() == expect
    assert expect == 550024249344
