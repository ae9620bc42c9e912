"""The lever manifest mirror (sched_rt.MANIFEST): the reference's row shape
(name, effect, min_sm, knob, disable sense, tag; python/sched_rt.py:72-79,
checked there against the C++ manifest by test/py/test_manifest.py:51-84),
and its order = the order in which the kernels apply the levers, read from
the kernel sources themselves: the claim loop (run_tasks) reads num_tasks
before it remaps a ticket through pi; each body reads the task's budget
before it picks the stream's policy, and commits the timer last."""
import os
import re

import pytest

import sched_rt

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "sched-pass_amd", "csrc")

# The reference's rows for the levers built here (python/sched_rt.py:72-79),
# name and effect only: the other fields describe its compile-time weave.
REFERENCE_ROWS = [("workqueue", "acquire"), ("pi", "E1/permute"), ("shed", "E2/budget"),
                  ("policy", "E0/hint"), ("timer", "O/observe")]


def src(name):
    with open(os.path.join(CSRC, name)) as f:
        return f.read()


def body(text, start):
    """The brace-balanced block that opens at the first '{' after `start`."""
    i = text.index("{", start)
    depth = 0
    for j in range(i, len(text)):
        depth += text[j] == "{"
        depth -= text[j] == "}"
        if depth == 0:
            return text[i:j + 1]
    raise AssertionError("unbalanced braces")


def first(text, pattern):
    m = re.search(pattern, text)
    assert m, pattern
    return m.start()


def test_rows_have_the_reference_shape():
    assert [(r[0], r[1]) for r in sched_rt.MANIFEST] == REFERENCE_ROWS
    for name, effect, min_sm, knob, disable, tag in sched_rt.MANIFEST:
        assert min_sm == 0 and knob is None and disable is False and tag == ""
        assert name in sched_rt.LEVER_ARMING


@pytest.mark.parametrize("header,loop", [
    ("levers.h", "__device__ __forceinline__ void run_tasks("),
    ("decode_wave.h", "__device__ __forceinline__ void run_wave_tasks("),
])
def test_claim_loops_acquire_before_they_remap(header, loop):
    text = src(header)
    run = body(text, text.index(loop))
    acquire = first(run, r"SCHED_CTRL_NUM_TASKS_OFF")
    remap = first(run, r"remap_wq\(|remap_static\(")
    assert acquire < remap


@pytest.mark.parametrize("kernel,entry", [
    ("decode_mfma.h", "__global__ void __launch_bounds__(NW * 64) decode_mfma("),
    ("decode_valu.h", "decode_valu(KParams P)"),
    ("decode_wave.h", "decode_wave(KParams P)"),
])
def test_kernel_bodies_apply_the_levers_in_manifest_order(kernel, entry):
    text = src(kernel)
    k = body(text, text.index(entry))
    # workqueue + pi: the body runs inside run_tasks (the wave kernel claims
    # per wave with its own loop, run_wave_tasks), which hands it the
    # remapped task; the wave kernel adds its timer row per wave (lt_timer)
    claim = first(k, r"run_tasks\(|run_wave_tasks<")
    shed = first(k, r"load_extent\(")
    timer = first(k, r"timer_commit\(|lt_timer\(")
    order = [claim, shed, timer]
    if kernel == "decode_mfma.h":           # the only kernel with a policy action
        order.insert(2, first(k, r"pol\.urgent"))
    assert order == sorted(order), (kernel, order)
    names = [r[0] for r in sched_rt.MANIFEST]
    assert names.index("workqueue") < names.index("pi") < names.index("shed") \
        < names.index("policy") < names.index("timer")
