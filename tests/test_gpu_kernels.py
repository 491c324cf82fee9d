"""Every kernel name on the MI355X against the CPU restatement, through the
C ABI (nlg_dispatch), on the seeded cases of tests/kernel_specs.py: bitwise
where the reference's result is a fixed sequence of integer or single f32
operations, and within the stated tolerance where a reduction's order or an
exp/pow/sin/cos differs.  Every buffer is compared after the run, outputs
and inputs alike (an input that changed is a bug too)."""
import sys

import numpy as np
import pytest

import kernel_specs as ks
import nlg_oracle as orc
import nlgpu
import np_ref

pytestmark = pytest.mark.gpu
CASES = ks.cases()


@pytest.fixture(scope="module", autouse=True)
def device():
    nlgpu.init()
    yield


def run_gpu(case):
    devs = []
    for i, b in enumerate(case.bufs):
        devs.append(devs[case.alias[i]] if i in case.alias else nlgpu.to_device(b))
    print(f"[gpu] {ks.case_id(case)} push={case.push} groups={case.groups}", flush=True)
    nlgpu.dispatch(case.name, [(d, case.bufs[i].size) for i, d in enumerate(devs)], case.push, case.groups)
    nlgpu.sync()
    return [d.download(np.float32, count=case.bufs[i].size) for i, d in enumerate(devs)]


def run_oracle(case):
    bufs = []
    for i, b in enumerate(case.bufs):
        bufs.append(bufs[case.alias[i]] if i in case.alias else np.array(b, copy=True))
    orc.dispatch(case.name, bufs, case.push, case.groups)
    return bufs


@pytest.mark.parametrize("case", CASES, ids=[ks.case_id(c) for c in CASES])
def test_kernel_matches_oracle(case):
    got = run_gpu(case)
    want = run_oracle(case)
    outs = set(np_ref.ref(case).keys())
    outs |= {i for i, j in case.alias.items() if j in outs} | {case.alias[i] for i in outs if i in case.alias}
    for i in range(len(case.bufs)):
        tol = case.tol if i in outs else ks.EXACT
        ok, err = np_ref.compare(got[i], want[i], tol)
        assert ok, f"{ks.case_id(case)} buffer {i}: error {err} (bar {tol})"


def test_short_buffer_is_rejected_before_launch():
    nlgpu.init()
    a = nlgpu.to_device(np.zeros(100, np.float32))
    c = nlgpu.to_device(np.zeros(100, np.float32))
    rc = nlgpu.dispatch("softmax", [a, (c, 50)], [1, 100], 1, check=False)
    assert rc != 0 and "needs" in nlgpu.last_error()
    rc = nlgpu.dispatch("no-such", [a], [1], 1, check=False)
    assert rc != 0 and "no kernel" in nlgpu.last_error()
    rc = nlgpu.dispatch("vadd", [a, c], [1], 1, check=False)
    assert rc != 0 and "buffers" in nlgpu.last_error()


def test_partial_grid_semantics():
    # groups*64 < domain: only the first 64*groups invocations run (vkserver dispatch)
    n = 300
    a = np.arange(n, dtype=np.float32)
    b = np.ones(n, np.float32)
    for groups in (1, 3):
        da, db, dc = nlgpu.to_device(a), nlgpu.to_device(b), nlgpu.to_device(np.full(n, -7, np.float32))
        nlgpu.dispatch("vadd", [da, db, dc], [n], groups)
        got = dc.download(count=n)
        k = min(n, 64 * groups)
        assert np.array_equal(got[:k], a[:k] + 1) and np.all(got[k:] == -7)
