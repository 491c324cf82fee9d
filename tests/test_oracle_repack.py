"""Weight ingest, CPU side: the oracle's repacking of the reference's int8-lane
(bitlinear-dp4a-1f/-rows, kernels.el:619-653) and base-4-in-float
(bitlinear-packed, kernels.el:992-1040) ternary weights into the 2-bit layout
of ternary-rows (kernels.el:700-746), pinned by known-answer words, by round
trips through packers and a 2-bit decoder written here independently of the
oracle, and by the reference's own linears giving the same results on either
form of the weights."""
import numpy as np
import pytest

import nlg_oracle as orc

f32 = np.float32


def decode2(w2, out, cols):
    """2-bit words -> values by sign extension (kernels.el:728-743)."""
    w = np.asarray(w2, np.uint32).reshape(out, -1)
    f = np.arange(cols)
    fields = (w[:, f // 16] >> (2 * (f % 16)).astype(np.uint32)) & 3
    return np.where(fields >= 2, fields.astype(np.int64) - 4, fields.astype(np.int64))


def pack_lanes(v):
    """int8 values [out x cols] -> lane words [out x ceil(cols/4)], lane l = column 4g+l."""
    out, cols = v.shape
    ng = (cols + 3) // 4
    b = np.zeros((out, 4 * ng), np.uint8)
    b[:, :cols] = v.astype(np.int8).view(np.uint8)
    return b.view("<u4").reshape(out, ng).copy()


def pack_base4(t, pk):
    """trits [out x cols] -> f32 values of pk base-4 codes (t+1), column f*pk+z = digit z."""
    out, cols = t.shape
    fcount = (cols + pk - 1) // pk
    codes = np.zeros((out, fcount * pk), np.int64)
    codes[:, :cols] = t + 1
    vals = (codes.reshape(out, fcount, pk) * (4 ** np.arange(pk))).sum(axis=2)
    assert vals.max() < 2 ** 24  # exact in f32
    return vals.astype(f32), fcount


def test_known_answer_words():
    # lanes [1, -1, 0, -2] -> fields 01, 11, 00, 10 -> 0b10_00_11_01
    w2, bad = orc.repack_i8_2bit(np.array([[0xFE00FF01]], np.uint32), 1, 4)
    assert bad == 0 and int(w2[0, 0]) == 0x8D
    # codes z=0..3 = 2, 0, 1, 2 (weights +1, -1, 0, +1) -> fields 01, 11, 00, 01
    v = f32(2 + 0 * 4 + 1 * 16 + 2 * 64)
    w2, bad = orc.repack_packed_2bit(np.array([[v]], f32), 1, 4, 4, 1)
    assert bad == 0 and int(w2[0, 0]) == 0b01_00_11_01


@pytest.mark.parametrize("out,cols", [(7, 37), (3, 4096), (5, 1), (2, 16), (4, 17)])
def test_int8_lanes_round_trip(out, cols):
    rng = np.random.default_rng(out * 1000 + cols)
    t = rng.integers(-2, 2, (out, cols))  # every 2-bit value, -2 included
    w2, bad = orc.repack_i8_2bit(pack_lanes(t), out, cols)
    assert bad == 0
    assert np.array_equal(decode2(w2, out, cols), t)
    # fields past cols stay zero
    if cols % 16:
        assert (np.asarray(w2)[:, -1] >> (2 * (cols % 16))).max() == 0


def test_int8_lanes_outside_the_code_are_zeroed_and_counted():
    v = np.array([[1, 2, -3, 127, -128, 0, -1, -2]])
    w2, bad = orc.repack_i8_2bit(pack_lanes(v), 1, 8)
    assert bad == 4
    assert decode2(w2, 1, 8).tolist() == [[1, 0, 0, 0, 0, 0, -1, -2]]


@pytest.mark.parametrize("out,cols,pk", [(5, 37, 12), (3, 2560, 12), (2, 100, 5), (4, 33, 1), (2, 48, 11)])
def test_base4_round_trip(out, cols, pk):
    rng = np.random.default_rng(out + cols + pk)
    t = rng.integers(-1, 2, (out, cols))
    vals, fcount = pack_base4(t, pk)
    w2, bad = orc.repack_packed_2bit(vals, out, cols, pk, fcount)
    assert bad == 0
    assert np.array_equal(decode2(w2, out, cols), t)


def test_base4_code3_and_missing_columns():
    # code 3 at z=1 -> counted, weight 0; fcount*pk < cols -> trailing columns carry no weight
    v = f32(2 + 3 * 4 + 0 * 16)  # codes 2, 3, 0 -> +1, bad, -1
    w2, bad = orc.repack_packed_2bit(np.array([[v]], f32), 1, 5, 3, 1)
    assert bad == 1
    assert decode2(w2, 1, 5).tolist() == [[1, 0, -1, 0, 0]]


def test_reference_linear_same_on_either_form():
    """bitlinear-dp4a-rows (kernels.el:636-653) on the int8 lanes and the
    composite 2-bit x int8 linear on the repacked words: same int32
    accumulators and epilogue, so the same bits."""
    seq, out, cols = 3, 37, 300
    rng = np.random.default_rng(5)
    t = rng.integers(-1, 2, (out, cols))
    wp = pack_lanes(t)
    w2, bad = orc.repack_i8_2bit(wp, out, cols)
    assert bad == 0
    x = rng.standard_normal(seq * cols).astype(f32)
    xq, g = orc.pack_act_rows(x, seq, cols)
    bias = rng.standard_normal(out).astype(f32)
    beta = (np.abs(rng.standard_normal(out)) * 0.05).astype(f32)
    y_ref = np.zeros(seq * out, f32)
    orc.dispatch("bitlinear-dp4a-rows", [xq.view(f32), wp.reshape(-1).view(f32), bias, beta, g, y_ref],
                 [seq, out, (cols + 3) // 4], (seq * out + 63) // 64)
    y = orc.ternary_linear_i8(xq, g, w2.reshape(-1), bias, beta, seq, out, cols, beta_per_row=True)
    assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32))


def test_packed_linear_matches_2bit_trits():
    """bitlinear-packed (f32 activations) on the base-4 weights equals the
    float64 sum over the trits the 2-bit words decode to (to f32 rounding)."""
    seq, out, cols, pk = 2, 9, 100, 12
    rng = np.random.default_rng(9)
    t = rng.integers(-1, 2, (out, cols))
    vals, fcount = pack_base4(t, pk)
    w2, _ = orc.repack_packed_2bit(vals, out, cols, pk, fcount)
    x = rng.standard_normal(seq * cols).astype(f32)
    bias = np.zeros(out, f32)
    beta = np.array([0.5], f32)
    y = np.zeros(seq * out, f32)
    orc.dispatch("bitlinear-packed", [x, vals.reshape(-1), bias, beta, y], [seq, cols, out, pk, fcount],
                 (seq * out + 63) // 64)
    want = x.reshape(seq, cols).astype(np.float64) @ (0.5 * decode2(w2, out, cols)).T
    assert np.abs(y.reshape(seq, out) - want).max() <= 1e-5 * max(1.0, np.abs(want).max())
