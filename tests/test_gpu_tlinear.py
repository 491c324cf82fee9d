"""The transposed linears on the MI355X (ternary-rows-t, dp4a-rows-t,
kernels.el:748-810) at the decoder's down-projection shape: bit-identical to
the CPU restatement (each column summed over the rows in the reference's
order), and adjoint to ternary-rows on the GPU (<W x, g> = <x, W' g>,
test/ternary-kernel-test.el:130-145)."""
import numpy as np
import pytest

import nlg_oracle as orc
import nlgpu

pytestmark = pytest.mark.gpu
f32 = np.float32


@pytest.fixture(scope="module", autouse=True)
def device():
    nlgpu.init()
    yield


def run(name, bufs, push, n):
    devs = [nlgpu.to_device(b) for b in bufs]
    nlgpu.dispatch(name, devs, push, (n + 63) // 64)
    return devs[-1].download(f32, bufs[-1].size)


@pytest.mark.parametrize("out,cols,seq", [(2560, 6912, 2), (6912, 2560, 1), (37, 300, 3)])
def test_ternary_rows_t_bit_exact(out, cols, seq):
    print(f"[gpu] ternary-rows-t out={out} cols={cols} seq={seq}", flush=True)
    rng = np.random.default_rng(out + cols)
    wng, nblk = (cols + 15) // 16, (cols + 127) // 128
    w = nlgpu.pack_ternary(nlgpu.trits(out + 7, (out, cols))).reshape(-1).view(f32)
    beta = (np.abs(rng.standard_normal(out * nblk)) * 0.05).astype(f32)
    g = rng.standard_normal(seq * out).astype(f32)
    x = np.zeros(seq * cols, f32)
    got = run("ternary-rows-t", [w, beta, g, x], [out, cols, nblk, wng, seq], seq * cols)
    want = x.copy()
    orc.dispatch("ternary-rows-t", [w.copy(), beta, g, want], [out, cols, nblk, wng, seq], (seq * cols + 63) // 64)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dp4a_rows_t_bit_exact():
    out, cols, seq = 2560, 2560, 2
    print(f"[gpu] dp4a-rows-t out={out} cols={cols} seq={seq}", flush=True)
    rng = np.random.default_rng(3)
    ng = (cols + 3) // 4
    w = rng.integers(0, 2 ** 32, out * ng, dtype=np.uint64).astype(np.uint32).view(f32)
    beta = (np.abs(rng.standard_normal(out)) * 0.05).astype(f32)
    g = rng.standard_normal(seq * out).astype(f32)
    x = np.zeros(seq * cols, f32)
    got = run("dp4a-rows-t", [w, beta, g, x], [out, cols, ng, seq], seq * cols)
    want = x.copy()
    orc.dispatch("dp4a-rows-t", [w.copy(), beta, g, want], [out, cols, ng, seq], (seq * cols + 63) // 64)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_adjoint_identity_on_gpu():
    seq, out, cols = 3, 2560, 6912
    nblk, wng = (cols + 127) // 128, (cols + 15) // 16
    rng = np.random.default_rng(20260921)
    w = nlgpu.pack_ternary(nlgpu.trits(5, (out, cols))).reshape(-1).view(f32)
    beta = (np.abs(rng.standard_normal(out * nblk)) * 0.05 + 0.01).astype(f32)
    x = rng.standard_normal(seq * cols).astype(f32)
    g = rng.standard_normal(seq * out).astype(f32)
    y = run("ternary-rows", [x, w, np.zeros(out, f32), beta, np.zeros(seq * out, f32)],
            [seq, out, cols, nblk, wng], seq * out)
    xt = run("ternary-rows-t", [w, beta, g, np.zeros(seq * cols, f32)], [out, cols, nblk, wng, seq], seq * cols)
    left, right = float(np.dot(y.astype(np.float64), g)), float(np.dot(x.astype(np.float64), xt))
    print(f"  <Wx,g> = {left:.6f}  <x,W'g> = {right:.6f}", flush=True)
    assert abs(left - right) <= 1e-5 * max(1e-6, abs(left))


@pytest.mark.parametrize("name,groups", [("ternary-rows-t", 7), ("dp4a-rows-t", 5)])
def test_rows_t_partial_grid(name, groups):
    """groups * 64 below seq * cols (a cut inside a position): only the first
    64 * groups outputs are written, bit-identical to the CPU restatement's,
    and the rest of X keeps its contents (the vkserver dispatch semantics)."""
    out, cols, seq = 70, 300, 3
    print(f"[gpu] {name} partial grid: out={out} cols={cols} seq={seq} groups={groups}", flush=True)
    rng = np.random.default_rng(groups)
    if name == "ternary-rows-t":
        wng, nblk = (cols + 15) // 16, (cols + 127) // 128
        w = nlgpu.pack_ternary(nlgpu.trits(11, (out, cols))).reshape(-1).view(f32)
        beta = (np.abs(rng.standard_normal(out * nblk)) * 0.05).astype(f32)
        push = [out, cols, nblk, wng, seq]
    else:
        ng = (cols + 3) // 4
        w = rng.integers(0, 2 ** 32, out * ng, dtype=np.uint64).astype(np.uint32).view(f32)
        beta = (np.abs(rng.standard_normal(out)) * 0.05).astype(f32)
        push = [out, cols, ng, seq]
    g = rng.standard_normal(seq * out).astype(f32)
    x = np.full(seq * cols, -7.0, f32)
    devs = [nlgpu.to_device(b) for b in (w, beta, g, x)]
    nlgpu.dispatch(name, devs, push, groups)
    got = devs[-1].download(f32, x.size)
    want = x.copy()
    orc.dispatch(name, [w.copy(), beta, g, want], push, groups)
    k = 64 * groups
    assert np.all(got[k:] == -7.0)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
