"""Row softmax on the MI355X (the config-3 operator: attention-score rows
~ N(0, 3^2) with -inf above the diagonal, max-subtracted, in place) against
the CPU restatement within 1e-5 relative per element, plus the properties
that hold at any size: rows sum to 1, masked entries are exactly 0."""
import numpy as np
import pytest

import nlg_oracle as orc
import nlgpu

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    nlgpu.init()
    yield


def causal_scores(seed, heads, n):
    a = nlgpu.normal(seed, heads * n * n, 3.0).reshape(heads, n, n)
    a[:, np.triu_indices(n, 1)[0], np.triu_indices(n, 1)[1]] = -np.inf
    return a.ravel()


@pytest.mark.parametrize("heads,n", [(2, 512), (1, 4096), (3, 1000), (1, 9000)])
@pytest.mark.parametrize("inplace", [False, True])
def test_softmax_matches_oracle(heads, n, inplace):
    print(f"[gpu] softmax heads={heads} n={n} inplace={inplace}", flush=True)
    a = causal_scores(heads * n, heads, n)
    rows = heads * n
    da = nlgpu.to_device(a)
    dc = da if inplace else nlgpu.DeviceArray(a.nbytes)
    nlgpu.softmax_rows(da, dc, rows, n)
    got = dc.download(np.float32, rows * n)
    want = orc.softmax_rows(a, rows, n)
    fin = want != 0
    assert np.array_equal(got == 0, want == 0)  # masked entries exactly 0
    rel = np.abs(got[fin].astype(np.float64) - want[fin]) / np.abs(want[fin])
    if n <= 4096:
        assert rel.max() <= 1e-5, rel.max()  # the bar, at the config-3 row width
    else:
        # Past 4096 columns the reference's own serial f32 sum drifts past
        # 1e-5 (its rounding error grows with the row), so the GPU is held to
        # 1e-5 against the exact softmax and to 1e-4 against the reference.
        assert rel.max() <= 1e-4, rel.max()
        r0 = slice(n * (n - 8), n * n)  # the last rows: ~n live entries each
        a64 = a[r0].reshape(8, n).astype(np.float64)
        e = np.exp(a64 - a64.max(axis=1, keepdims=True))
        exact = (e / e.sum(axis=1, keepdims=True)).ravel()
        live = exact > 0
        rel_exact = np.abs(got[r0][live] - exact[live]) / exact[live]
        assert rel_exact.max() <= 1e-5, rel_exact.max()
    sums = got.reshape(rows, n).astype(np.float64).sum(axis=1)
    assert np.abs(sums - 1).max() < 1e-4
