"""The decode hot path on the MI355X: pack-act-rows quantisation and the
2-bit x int8 ternary linear, bit-exact against the CPU restatement (exact
int32 accumulators and the same IEEE epilogue), at the BASELINE shapes
(4096 x 4096 decode GEMV; the 2560/6912 SwiGLU projections at B = 1 and
16) and at ragged edges (cols not a multiple of 16 or 4, one row, one
column), for every launch geometry."""
import numpy as np
import pytest

import nlg_oracle as orc
import nlgpu

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    nlgpu.init()
    yield


def make(seed, seq, out, cols, per_row=False):
    t = nlgpu.trits(seed, (out, cols))
    w2 = nlgpu.pack_ternary(t)
    x = nlgpu.normal(seed + 1, seq * cols)
    bias = nlgpu.normal(seed + 2, out) * np.float32(0.1)
    beta = (np.abs(nlgpu.normal(seed + 3, out if per_row else 1)) * np.float32(0.05)).astype(np.float32)
    return t, w2, x, bias, beta


SHAPES = [(1, 4096, 4096), (1, 6912, 2560), (1, 2560, 6912), (16, 6912, 2560), (16, 2560, 6912),
          (3, 37, 300), (1, 100, 1000), (2, 33, 4100), (5, 64, 16), (1, 1, 64), (4, 7, 1), (1, 5, 17),
          (9, 130, 2048)]


@pytest.mark.parametrize("seq,out,cols", SHAPES)
def test_pack_and_ternary_linear_bit_exact(seq, out, cols):
    print(f"[gpu] ternary seq={seq} out={out} cols={cols}", flush=True)
    t, w2, x, bias, beta = make(seq * 7 + cols, seq, out, cols)
    ng = (cols + 3) // 4
    dx = nlgpu.to_device(x)
    dxq = nlgpu.DeviceArray(seq * ng * 4)
    dg = nlgpu.DeviceArray(seq * 4)
    nlgpu.pack_act_rows(dx, dxq, dg, seq, cols)
    xq_ref, g_ref = orc.pack_act_rows(x, seq, cols)
    nlgpu.sync()
    assert np.array_equal(dxq.download(np.uint32, seq * ng), xq_ref)
    assert np.array_equal(dg.download(np.float32, seq).view(np.uint32), g_ref.view(np.uint32))
    dw, db, dbe = nlgpu.to_device(w2), nlgpu.to_device(bias), nlgpu.to_device(beta)
    dy = nlgpu.DeviceArray(seq * out * 4)
    nlgpu.ternary_linear_i8(dxq, dg, dw, db, dbe, dy, seq, out, cols)
    y = dy.download(np.float32, seq * out)
    y_ref = orc.ternary_linear_i8(xq_ref, g_ref, w2, bias, beta, seq, out, cols)
    bad = np.flatnonzero(y.view(np.uint32) != y_ref.view(np.uint32))
    assert bad.size == 0, f"{bad.size} outputs differ, first {bad[:5]}: {y[bad[:3]]} vs {y_ref[bad[:3]]}"


@pytest.mark.parametrize("rpw", [1, 2, 4, 8])
@pytest.mark.parametrize("wpb", [1, 2, 4])
def test_every_launch_geometry_gives_the_same_bits(rpw, wpb):
    seq, out, cols = 2, 1027, 2560
    t, w2, x, bias, beta = make(99, seq, out, cols, per_row=True)
    xq, g = orc.pack_act_rows(x, seq, cols)
    y_ref = orc.ternary_linear_i8(xq, g, w2, None, beta, seq, out, cols, beta_per_row=True)
    dy = nlgpu.DeviceArray(seq * out * 4)
    nlgpu.ternary_linear_i8(nlgpu.to_device(xq), nlgpu.to_device(g), nlgpu.to_device(w2), None,
                            nlgpu.to_device(beta), dy, seq, out, cols, beta_per_row=True,
                            rows_per_wave=rpw, waves_per_block=wpb)
    assert np.array_equal(dy.download(np.float32, seq * out).view(np.uint32), y_ref.view(np.uint32))


def test_named_ternary_i8_matches_typed_entry():
    seq, out, cols = 3, 300, 1024
    t, w2, x, bias, beta = make(5, seq, out, cols)
    xq, g = orc.pack_act_rows(x, seq, cols)
    y_ref = orc.ternary_linear_i8(xq, g, w2, bias, beta, seq, out, cols)
    dy = nlgpu.DeviceArray(seq * out * 4)
    bufs = [nlgpu.to_device(xq), nlgpu.to_device(w2), nlgpu.to_device(bias), nlgpu.to_device(beta),
            nlgpu.to_device(g), dy]
    nlgpu.dispatch("ternary-i8", bufs, [seq, out, cols], (seq * out + 63) // 64)
    assert np.array_equal(dy.download(np.float32, seq * out).view(np.uint32), y_ref.view(np.uint32))


@pytest.mark.parametrize("groups", [1, 7, 15])
def test_named_ternary_i8_partial_grid(groups):
    """groups*64 < seq*out: invocations idx = s*out + o < 64*groups write
    their outputs, the rest of Y keeps its contents (whole rows, then part of
    the next row)."""
    seq, out, cols = 4, 300, 1024
    t, w2, x, bias, beta = make(6, seq, out, cols)
    xq, g = orc.pack_act_rows(x, seq, cols)
    y_ref = orc.ternary_linear_i8(xq, g, w2, bias, beta, seq, out, cols)
    y0 = np.full(seq * out, -3.5, np.float32)
    dy = nlgpu.to_device(y0)
    bufs = [nlgpu.to_device(xq), nlgpu.to_device(w2), nlgpu.to_device(bias), nlgpu.to_device(beta),
            nlgpu.to_device(g), dy]
    nlgpu.dispatch("ternary-i8", bufs, [seq, out, cols], groups)
    n = min(seq * out, 64 * groups)
    got = dy.download(np.float32, seq * out)
    assert np.array_equal(got[:n].view(np.uint32), y_ref[:n].view(np.uint32))
    assert np.all(got[n:] == -3.5)


def test_int32_accumulator_extremes():
    # every weight -2 (code 10) against x = +-127 lanes: the largest partial sums
    seq, out, cols = 2, 64, 8192
    t = np.full((out, cols), -2, np.int8)
    t[1::2, ::3] = 1
    w2 = nlgpu.pack_ternary(t)
    x = np.full(seq * cols, 5.0, np.float32)
    x[cols:] = -5.0  # second token all -127 lanes
    xq, g = orc.pack_act_rows(x, seq, cols)
    acc = orc.ternary_acc_i8(xq, w2, seq, out, cols)
    assert np.abs(acc).max() > 100000
    y_ref = orc.ternary_linear_i8(xq, g, w2, None, np.array([1.0], np.float32), seq, out, cols)
    dy = nlgpu.DeviceArray(seq * out * 4)
    nlgpu.ternary_linear_i8(nlgpu.to_device(xq), nlgpu.to_device(g), nlgpu.to_device(w2), None,
                            nlgpu.to_device(np.array([1.0], np.float32)), dy, seq, out, cols)
    assert np.array_equal(dy.download(np.float32, seq * out).view(np.uint32), y_ref.view(np.uint32))


FUSED = [(1, 4096, 4096), (1, 6912, 2560), (1, 2560, 6912), (2, 3840, 2560), (3, 100, 1024), (3, 5, 64),
         (4, 100, 960), (1, 128256, 2560)]


@pytest.mark.parametrize("seq,out,cols", FUSED)
@pytest.mark.parametrize("rpw", [0, 1, 2, 4])
def test_fused_linear_bit_exact(seq, out, cols, rpw):
    if rpw and out > 20000:
        pytest.skip("geometry sweep on the small shapes only")
    print(f"[gpu] fused ternary seq={seq} out={out} cols={cols} rpw={rpw}", flush=True)
    t, w2, x, bias, beta = make(seq * 3 + out, seq, out, cols, per_row=(out % 2 == 0))
    xq, g = orc.pack_act_rows(x, seq, cols)
    y_ref = orc.ternary_linear_i8(xq, g, w2, bias, beta, seq, out, cols, beta_per_row=(out % 2 == 0))
    dy, dg = nlgpu.DeviceArray(seq * out * 4), nlgpu.DeviceArray(seq * 4)
    nlgpu.ternary_linear(nlgpu.to_device(x), nlgpu.to_device(w2), nlgpu.to_device(bias), nlgpu.to_device(beta),
                         dy, seq, out, cols, beta_per_row=(out % 2 == 0), gamma_out=dg, rows_per_wave=rpw)
    assert np.array_equal(dg.download(np.float32, seq).view(np.uint32), g.view(np.uint32))
    assert np.array_equal(dy.download(np.float32, seq * out).view(np.uint32), y_ref.view(np.uint32))


BATCHED = [(4, 100, 1024), (6, 2560, 6912), (7, 3840, 2560), (8, 64, 256), (16, 300, 2560), (17, 2560, 2560), (32, 13824, 2560), (33, 2560, 6912),
           (64, 512, 4096), (100, 256, 1024), (512, 2560, 2560), (512, 6912, 2560),
           (200, 1000, 512), (600, 16448, 256),  # 64-row tiles, ragged; 128-row tiles, ragged
           (40, 16400, 512), (32, 8200, 768),  # enough 64-row workgroups: the unsplit small-batch kernel
           (24, 1000, 12288), (9, 130, 8192),  # split columns, 12 and 8 chunks per wave (the 16-chunk form)
           # 1,024+ 64-row tiles of <= 2,560 columns: resident activations, a
           # loop over row tiles (16 and 32 tokens, ragged rows, two token
           # blocks, rows shorter than the 10-chunk stage)
           (20, 65600, 512), (9, 66001, 2560), (40, 33000, 256)]


@pytest.mark.parametrize("seq,out,cols", BATCHED)
def test_batched_matrix_core_linear_bit_exact(seq, out, cols):
    """4+ tokens and cols % 256 == 0: per-token quantisation, then the int8
    MFMA GEMM; same int32 accumulators and epilogue bits as the reference."""
    print(f"[gpu] batched ternary seq={seq} out={out} cols={cols}", flush=True)
    per_row = out % 2 == 0
    t, w2, x, bias, beta = make(seq * 5 + out + cols, seq, out, cols, per_row=per_row)
    xq, g = orc.pack_act_rows(x, seq, cols)
    y_ref = orc.ternary_linear_i8(xq, g, w2, bias, beta, seq, out, cols, beta_per_row=per_row)
    dy, dg = nlgpu.DeviceArray(seq * out * 4), nlgpu.DeviceArray(seq * 4)
    nlgpu.ternary_linear(nlgpu.to_device(x), nlgpu.to_device(w2), nlgpu.to_device(bias), nlgpu.to_device(beta),
                         dy, seq, out, cols, beta_per_row=per_row, gamma_out=dg)
    assert np.array_equal(dg.download(np.float32, seq).view(np.uint32), g.view(np.uint32))
    y = dy.download(np.float32, seq * out)
    bad = np.flatnonzero(y.view(np.uint32) != y_ref.view(np.uint32))
    assert bad.size == 0, f"{bad.size} differ, first {bad[:5]}: {y[bad[:3]]} vs {y_ref[bad[:3]]}"
    if out >= 32768:  # the resident-activation GEMM again, on a registered tiled copy
        dw = nlgpu.to_device(w2)
        nlgpu.ternary_tiled_register(dw, out, cols)
        try:
            dy.zero()
            nlgpu.ternary_linear(nlgpu.to_device(x), dw, nlgpu.to_device(bias), nlgpu.to_device(beta),
                                 dy, seq, out, cols, beta_per_row=per_row)
        finally:
            nlgpu.ternary_tiled_unregister(dw)
        y = dy.download(np.float32, seq * out)
        assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32)), "tiled copy"


@pytest.mark.parametrize("seq,out,cols", [(16, 300, 2496), (2, 50, 1000), (5, 64, 4032)])
def test_linear_two_launch_path_with_workspace(seq, out, cols):
    t, w2, x, bias, beta = make(77 + seq, seq, out, cols)
    xq, g = orc.pack_act_rows(x, seq, cols)
    y_ref = orc.ternary_linear_i8(xq, g, w2, bias, beta, seq, out, cols)
    dy = nlgpu.DeviceArray(seq * out * 4)
    dx, dw, db, dbe = (nlgpu.to_device(a) for a in (x, w2, bias, beta))
    with pytest.raises(nlgpu.NlgError):
        nlgpu.ternary_linear(dx, dw, db, dbe, dy, seq, out, cols)  # needs a workspace
    ws = nlgpu.DeviceArray(nlgpu.ternary_linear_workspace(seq, cols))
    nlgpu.ternary_linear(dx, dw, db, dbe, dy, seq, out, cols, workspace=ws)
    assert np.array_equal(dy.download(np.float32, seq * out).view(np.uint32), y_ref.view(np.uint32))


def test_batched_linears_on_two_streams_do_not_share_scratch():
    """Batched calls (per-token quantisation into library scratch, then the
    GEMM) issued back to back on two streams may overlap; each stream has
    its own scratch, so both give the single-stream bits."""
    seq, out, cols = 64, 2560, 2560
    streams = [nlgpu.lib().nlg_stream_create() for _ in range(2)]
    cases, want = [], []
    for i in range(2):
        t, w2, x, bias, beta = make(1000 + i, seq, out, cols)
        xq, g = orc.pack_act_rows(x, seq, cols)
        want.append(orc.ternary_linear_i8(xq, g, w2, bias, beta, seq, out, cols))
        cases.append([nlgpu.to_device(a) for a in (x, w2, bias, beta)] + [nlgpu.DeviceArray(seq * out * 4)])
    nlgpu.sync()
    for rep in range(20):  # interleaved: stream 0's quantisation can land between stream 1's
        for i in (0, 1):
            dx, dw, db, dbe, dy = cases[i]
            nlgpu.ternary_linear(dx, dw, db, dbe, dy, seq, out, cols, stream=streams[i])
    for st in streams:
        nlgpu.sync(st)
    for i in (0, 1):
        assert np.array_equal(cases[i][4].download(np.uint32, seq * out), want[i].view(np.uint32)), i
    for st in streams:
        nlgpu.lib().nlg_stream_destroy(st)


def test_timed_linear_matches_and_stamps():
    """The measurement variant (nlg_ternary_linear_timed) computes the same
    bits as the plain linear and leaves one (start, end) wall-clock pair per
    wave, end after start, all within one launch's span."""
    out, cols = 4096, 4096
    w2 = nlgpu.pack_ternary(nlgpu.trits(77, (out, cols)))
    x = nlgpu.normal(78, cols)
    beta = np.array([0.03], np.float32)
    dx, dw, db = nlgpu.to_device(x), nlgpu.to_device(w2), nlgpu.to_device(beta)
    y0, y1 = nlgpu.DeviceArray(out * 4), nlgpu.DeviceArray(out * 4)
    nlgpu.ternary_linear(dx, dw, None, db, y0, 1, out, cols)
    L = nlgpu.lib()
    nst = int(L.nlg_ternary_linear_timed_stamps(out))
    assert nst == 256 * 4 * 16
    ds = nlgpu.DeviceArray(nst)
    assert L.nlg_ternary_linear_timed(dx.ptr, dw.ptr, db.ptr, y1.ptr, out, cols, ds.ptr, nst, None) == 0
    nlgpu.sync()
    a, b = y0.download(np.float32, out), y1.download(np.float32, out)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    st = ds.download(np.uint64, nst // 8).reshape(-1, 2).astype(np.int64)
    assert np.all(st[:, 0] > 0) and np.all(st[:, 1] >= st[:, 0])
    span = (st[:, 1].max() - st[:, 0].min()) / 100.0  # us at 100 MHz
    assert 0.0 < span < 1000.0, span
    with pytest.raises(nlgpu.NlgError, match="short"):
        nlgpu._check(L.nlg_ternary_linear_timed(dx.ptr, dw.ptr, db.ptr, y1.ptr, out, cols, ds.ptr, nst - 16, None),
                     "timed")
