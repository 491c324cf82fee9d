"""nlg_ternary_linear_noalloc (its scratch in the library's fixed device
array) against nlg_ternary_linear (a caller workspace, or the library's
per-stream scratch): the same bits, on each of the three forms the linear
takes, for two calls in a row with the second smaller than the first (the
array keeps the first call's contents), and a clear error, with nothing
launched, for a shape whose scratch exceeds the array."""
import numpy as np
import pytest

import nlgpu

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    nlgpu.init()
    yield


def case(seed, seq, out, cols):
    w2 = nlgpu.pack_ternary(nlgpu.trits(seed, (out, cols)))
    x = nlgpu.normal(seed + 1, seq * cols)
    bias = (nlgpu.normal(seed + 2, out) * np.float32(0.1)).astype(np.float32)
    beta = (np.abs(nlgpu.normal(seed + 3, out)) * np.float32(0.05)).astype(np.float32)
    return [nlgpu.to_device(a) for a in (x, w2, bias, beta)]


def run_both(seed, seq, out, cols):
    dx, dw, db, dbe = case(seed, seq, out, cols)
    ws = nlgpu.DeviceArray(nlgpu.ternary_linear_workspace(seq, cols))
    y0, g0 = nlgpu.DeviceArray(seq * out * 4), nlgpu.DeviceArray(seq * 4)
    y1, g1 = nlgpu.DeviceArray(seq * out * 4), nlgpu.DeviceArray(seq * 4)
    nlgpu.ternary_linear(dx, dw, db, dbe, y0, seq, out, cols, beta_per_row=True, gamma_out=g0, workspace=ws)
    nlgpu.ternary_linear_noalloc(dx, dw, db, dbe, y1, seq, out, cols, beta_per_row=True, gamma_out=g1)
    a, b = y0.download(np.uint32, seq * out), y1.download(np.uint32, seq * out)
    assert np.array_equal(a, b), f"{np.sum(a != b)} of {a.size} outputs differ"
    assert np.array_equal(g0.download(np.uint32, seq), g1.download(np.uint32, seq))


# (first, second): the second call smaller than the first, on the same form
FORMS = {
    "batched matrix-core": ((512, 2560, 2560), (100, 640, 1024)),
    "two launches": ((40, 300, 1000), (6, 300, 1000)),
    "one launch": ((3, 4096, 4096), (1, 2560, 2560)),
}


@pytest.mark.parametrize("form", list(FORMS))
def test_noalloc_linear_equals_workspace_linear(form):
    for i, (seq, out, cols) in enumerate(FORMS[form]):
        print(f"[gpu] noalloc linear {form} call {i}: seq={seq} out={out} cols={cols}", flush=True)
        run_both(seq * 3 + cols + i, seq, out, cols)


def test_noalloc_rejects_a_shape_beyond_the_fixed_scratch():
    seq, out, cols = 8192, 64, 4096  # 32 MiB of int8 activations
    assert seq * cols > 16 << 20
    dx, dw, db, dbe = case(5, 8, out, cols)  # never read: the call must fail first
    with pytest.raises(nlgpu.NlgError, match="fixed"):
        nlgpu.ternary_linear_noalloc(dx, dw, db, dbe, dx, seq, out, cols)
