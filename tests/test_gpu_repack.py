"""Weight ingest on the MI355X: the int8-lane and base-4-in-float ternary
weights repacked into the 2-bit layout, bit for bit as the CPU restatement
(including the count of weights the 2-bit code cannot hold), and the
reference's bitlinear-dp4a-rows on the original lanes equal to the 2-bit
linear on the repacked words."""
import numpy as np
import pytest

import nlg_oracle as orc
import nlgpu
from test_oracle_repack import pack_base4, pack_lanes

pytestmark = pytest.mark.gpu
f32 = np.float32


@pytest.fixture(scope="module", autouse=True)
def device():
    nlgpu.init()
    yield


@pytest.mark.parametrize("out,cols", [(13824, 2560), (37, 300), (5, 1), (3, 17), (2560, 6912)])
def test_repack_int8_lanes_bit_exact(out, cols):
    print(f"[gpu] repack int8 lanes out={out} cols={cols}", flush=True)
    rng = np.random.default_rng(out + cols)
    v = rng.integers(-1, 2, (out, cols))
    v[rng.random((out, cols)) < 0.001] = 5  # a few unrepresentable lanes
    v[rng.random((out, cols)) < 0.001] = -2
    wp = pack_lanes(v)
    want, bad = orc.repack_i8_2bit(wp, out, cols)
    w2 = nlgpu.DeviceArray(want.nbytes)
    nbad = nlgpu.to_device(np.zeros(1, np.uint32))
    nlgpu.repack_i8_to_2bit(nlgpu.to_device(wp), out, cols, w2, nbad)
    assert np.array_equal(w2.download(np.uint32, want.size), want.reshape(-1))
    assert int(nbad.download(np.uint32, 1)[0]) == bad


@pytest.mark.parametrize("out,cols,pk", [(6912, 2560, 12), (37, 300, 12), (5, 96, 12), (3, 48, 12),
                                         (4, 33, 1), (2, 48, 16), (9, 100, 5)])
def test_repack_base4_bit_exact(out, cols, pk):
    print(f"[gpu] repack base-4 out={out} cols={cols} pk={pk}", flush=True)
    rng = np.random.default_rng(out * pk + cols)
    t = rng.integers(-1, 2, (out, cols))
    vals, fcount = pack_base4(t, pk) if pk <= 12 else (None, None)
    if vals is None:  # 16 codes overflow f32's exact range: random bit patterns instead
        fcount = (cols + pk - 1) // pk
        vals = rng.integers(0, 2 ** 24, (out, fcount)).astype(f32)
    vals[rng.random(vals.shape) < 0.01] = f32(3 * 4 ** (pk // 2))  # code 3 somewhere
    if fcount > 1:
        fcount -= 1  # the last columns carry no weight
        vals = np.ascontiguousarray(vals[:, :fcount])
    want, bad = orc.repack_packed_2bit(vals, out, cols, pk, fcount)
    w2 = nlgpu.DeviceArray(want.nbytes)
    nbad = nlgpu.to_device(np.zeros(1, np.uint32))
    nlgpu.repack_packed_to_2bit(nlgpu.to_device(vals), out, cols, pk, fcount, w2, nbad)
    assert np.array_equal(w2.download(np.uint32, want.size), want.reshape(-1))
    assert int(nbad.download(np.uint32, 1)[0]) == bad


def test_dp4a_rows_equals_2bit_linear_after_repack():
    seq, out, cols = 5, 2560, 2560
    print(f"[gpu] dp4a-rows vs repacked 2-bit linear seq={seq} out={out} cols={cols}", flush=True)
    rng = np.random.default_rng(11)
    t = rng.integers(-1, 2, (out, cols))
    wp = pack_lanes(t)
    x = rng.standard_normal(seq * cols).astype(f32)
    bias = rng.standard_normal(out).astype(f32)
    beta = (np.abs(rng.standard_normal(out)) * 0.05).astype(f32)
    xq, g = orc.pack_act_rows(x, seq, cols)
    dxq, dg, dwp = nlgpu.to_device(xq), nlgpu.to_device(g), nlgpu.to_device(wp)
    dbias, dbeta = nlgpu.to_device(bias), nlgpu.to_device(beta)
    y_ref = nlgpu.DeviceArray(seq * out * 4)
    nlgpu.dispatch("bitlinear-dp4a-rows", [dxq, dwp, dbias, dbeta, dg, y_ref], [seq, out, (cols + 3) // 4],
                   (seq * out + 63) // 64)
    w2 = nlgpu.DeviceArray(out * ((cols + 15) // 16) * 4)
    nlgpu.repack_i8_to_2bit(dwp, out, cols, w2)
    y = nlgpu.DeviceArray(seq * out * 4)
    nlgpu.ternary_linear_i8(dxq, dg, w2, dbias, dbeta, y, seq, out, cols, beta_per_row=True)
    a, b = y.download(f32, seq * out), y_ref.download(f32, seq * out)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
