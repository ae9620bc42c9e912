"""bench.py's contract pieces that run without a GPU: more than one GPU is
refused with a message (one GPU per run), the fixture generator matches the
reference fixtures' LCG step by step, and the argument defaults."""
import os
import subprocess
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_fixture_generator_matches_the_lcg_loop():
    from bench import _lcg_uniform
    s, ref = 777, []
    for _ in range(9000):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        ref.append(((s >> 8) & 0xFFFF) / 65536.0 - 0.5)
    ref = np.array(ref, np.float32)
    for n in (1, 4095, 4096, 4097, 9000):
        assert np.array_equal(_lcg_uniform(n, 777), ref[:n]), n


def test_default_sections_and_steps():
    import bench
    old = sys.argv
    try:
        sys.argv = ["bench.py"]
        a = bench.parse()
    finally:
        sys.argv = old
    assert a.gpus == 1 and a.steps > 0 and a.warmup >= 0
    assert set(a.sections.split(",")) >= {"hetero", "shed", "fp8", "kv", "trace", "fixture"}
