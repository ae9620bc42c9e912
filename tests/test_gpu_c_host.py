"""A C++ host program (tests/c_host/paged_decode_host.cpp) of the kind that
included the reference's runtime/sched_rt.h: it links libschedpd.so, arms
the levers through the sched_rt_* C ABI and launches sched_paged_decode with
the levers from the __sched_* slots (test/paged_decode.cu:255-380's flow).
Its outputs against the oracle: the stock decode within tolerance; the
armed-neutral, reversed-pi, timed and ticket-queue launches bitwise equal to
it, one nonzero timer row per task; per-task shed budgets against the
truncated oracle."""
import os
import subprocess

import numpy as np
import pytest
import torch

import oracle
import workloads
from parity import TOL_BF16, par_err
from sched_rt import SchedPlane

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST = os.path.join(ROOT, "tests", "c_host", "paged_decode_host")


def test_cpp_host_program_drives_the_levers_through_the_c_abi(tmp_path):
    assert os.path.exists(HOST), "tests/c_host/paged_decode_host is not built: run " \
                                 "__graft_entry__.build() (make -C tests/c_host)"
    ctx = [1, 16, 300, 2048, 777, 3000, 64, 1500]
    R, hq, hkv, d, ps = len(ctx), 32, 8, 128, 16
    b = workloads.make_batch(np.asarray(ctx), num_q_heads=hq, num_kv_heads=hkv, head_dim=d,
                             kv_dtype=torch.bfloat16, q_dtype=torch.bfloat16, seed=31,
                             device="cpu")
    bt = b["block_table"].numpy().astype(np.int32)
    pages = b["k_pool"].shape[0]
    ntask = R * hkv
    tau = np.random.default_rng(5).integers(0, 2500, ntask).astype(np.uint16)
    tau[::3] = 0
    W = 7
    with open(tmp_path / "meta.txt", "w") as f:
        f.write(f"{R} {hq} {hkv} {d} {ps} {bt.shape[1]} {pages} {W}\n")
    for name, t in (("q", b["q"]), ("k", b["k_pool"]), ("v", b["v_pool"])):
        t.contiguous().view(torch.int16).numpy().tofile(tmp_path / f"{name}.bin")
    bt.tofile(tmp_path / "bt.bin")
    b["ctx_lens"].numpy().astype(np.int32).tofile(tmp_path / "ctx.bin")
    tau.tofile(tmp_path / "tau.bin")
    print("running the C++ host program", flush=True)
    p = subprocess.run([HOST, str(tmp_path)], capture_output=True, text=True, timeout=120)
    print(p.stdout, p.stderr, flush=True)
    assert p.returncode == 0 and p.stdout.strip().endswith("ok"), p.stderr

    def out(mode):
        return np.fromfile(tmp_path / f"out_{mode}.bin", np.float32).reshape(R, hq, d)

    stock = out("stock")
    ref = oracle.decode(b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"])
    assert par_err(stock, ref, "C++ host, stock") <= TOL_BF16
    for mode in ("neutral", "reversed", "timed", "queue"):
        assert np.array_equal(out(mode), stock), mode
    rows = np.fromfile(tmp_path / "timer.bin", np.uint64)
    assert rows.size == ntask and (rows > 0).all()
    plane = SchedPlane(max_tasks=4096, device="cpu")
    plane.set_rows(tau=tau.astype(np.int64), n=ntask)
    shed_ref = oracle.decode(b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"],
                             ctrl=bytes(plane._ctrl_host), max_tasks=4096)
    assert par_err(out("shed"), shed_ref, "C++ host, shed") <= TOL_BF16
    assert not np.allclose(out("shed"), stock)            # the budgets cut something
