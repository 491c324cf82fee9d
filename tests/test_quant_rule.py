"""The division-free exact quantisation of the GPU kernels (lane_q8 /
quant_word in nelisp-gpu_amd/csrc/nlg_quant.h) against the reference's
rounding (pack-act-rows, lisp/nelisp-gpu-kernels.el:912-926:
q = RN(v/g), ri = min(trunc(RN(|q| + 0.5)), 127), byte = ri or
(256 - ri) % 256 when q < 0), both restated in numpy.

The kernels form g = RN(amax/127) (itself by one correction step of the
constant RN(1/127)) and y = RN(1/g) once per row, and per element take
q0 = RN(v*y), r = fma(-q0, g, v), q = fma(r, y, q0) -- one correction step
of the reciprocal product -- then trunc(RN(q + copysign(0.5, v))) clamped to
+-127.  The claim under test is that q is exactly the correctly rounded
quotient for every v once g >= 2^-90 (rows below that divide per element),
so every byte equals the reference's.  fma is restated exactly: the product
of two float32 values is exact in float64, the sum's rounding error is
recovered by a two-sum, and an exact float32 midpoint is resolved by that
error's sign.  Checked on random rows across 55 decades of scale, on values
walked ulp by ulp across every rounding boundary k + 1/2 (where a wrong
quotient would flip a byte), and on the special values; a planted error (the
correction step dropped) is shown to fail.  CPU only.
"""
import numpy as np

f32, f64 = np.float32, np.float64
FAST_MIN = f32(2.0 ** -90)


def fmaf(a, b, c):
    """Correctly rounded float32 a*b + c."""
    a, b, c = np.asarray(a, f32), np.asarray(b, f32), np.asarray(c, f32)
    p = a.astype(f64) * b.astype(f64)  # exact: 24 + 24 bits
    cc = c.astype(f64)
    with np.errstate(all="ignore"):
        s = p + cc
        bb = s - p
        e = (p - (s - bb)) + (cc - bb)  # s + e == p + c exactly
        f = s.astype(f32)
        diff = s - f.astype(f64)
        nb = np.nextafter(f, np.where(diff > 0, f32(np.inf), f32(-np.inf)).astype(f32))
        mid = (f.astype(f64) + nb.astype(f64)) * 0.5
    away = (diff != 0) & (s == mid) & (e != 0) & (np.sign(e) == np.sign(diff))
    return np.where(away, nb, f)


def reference_byte(v, g):
    """pack-act-rows, statement by statement (IEEE float32 division)."""
    v = np.asarray(v, f32)
    with np.errstate(all="ignore"):
        q = (v / g).astype(f32) if g > 0 else np.zeros_like(v)
        neg = q < 0
        aq = np.where(neg, (f32(0.0) - q).astype(f32), q)
        t = (aq + f32(0.5)).astype(f32)
        ri = np.where(np.isnan(t), 0, np.minimum(np.trunc(np.nan_to_num(t, posinf=1e9)), 127)).astype(np.int64)
    return np.where(neg, (256 - ri) % 256, ri)


def kernel_quotient(v, g, correct=True):
    ginv = (f32(1.0) / g).astype(f32)
    with np.errstate(all="ignore"):
        q0 = (v * ginv).astype(f32)
    if not correct:
        return q0
    return fmaf(fmaf(-q0, g, v), ginv, q0)


def kernel_byte(v, g, correct=True):
    v = np.asarray(v, f32)
    if not (g >= FAST_MIN and np.isfinite(g)):
        return reference_byte(v, g)  # the per-element division path
    q = kernel_quotient(v, g, correct)
    with np.errstate(all="ignore"):
        s = (q + np.copysign(f32(0.5), v).astype(f32)).astype(f32)
        t = np.where(np.isnan(s), 0, np.trunc(np.nan_to_num(s))).astype(np.int64)  # v_cvt_i32_f32
    return np.clip(t, -127, 127) % 256


def check(v, g, correct=True):
    v = np.asarray(v, f32)
    g = f32(g)
    want = reference_byte(v, g)
    got = kernel_byte(v, g, correct)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, (v[bad[:5]], got[bad[:5]], want[bad[:5]])


def boundary_walk(g, ulps=24):
    centre = ((np.arange(0, 129, dtype=f64) + 0.5) * f64(g)).astype(f32)
    out, up, down = [centre], centre.copy(), centre.copy()
    for _ in range(ulps):
        up = np.nextafter(up, f32(np.inf))
        down = np.nextafter(down, f32(0))
        out += [up, down]
    v = np.concatenate(out)
    return np.concatenate([v, -v])


def test_quotient_is_the_ieee_division():
    rng = np.random.default_rng(2024)
    for _ in range(40):
        g = f32(f32(10.0 ** rng.uniform(-25, 30)) * f32(rng.uniform(1, 2)))
        v = (rng.uniform(-127, 127, 100_000) * f64(g)).astype(f32)
        with np.errstate(all="ignore"):
            assert np.array_equal(kernel_quotient(v, g), (v / g).astype(f32))


def test_random_rows():
    rng = np.random.default_rng(2024)
    for _ in range(20):
        amax = f32(10.0 ** rng.uniform(-30, 30))
        g = f32(amax / f32(127.0))
        v = (rng.uniform(-1, 1, 200_000) * amax).astype(f32)
        v[:2] = [amax, -amax]
        check(v, g)


def test_every_rounding_boundary():
    rng = np.random.default_rng(7)
    scales = [f32(f32(10.0 ** rng.uniform(-25, 25)) * f32(rng.uniform(1, 2))) for _ in range(60)]
    scales += [f32(1.0), f32(2.0 ** -20), np.nextafter(f32(2.0), f32(0)), FAST_MIN,
               np.nextafter(FAST_MIN, f32(0)), f32(2.0 ** -126), f32(2.0 ** -127), f32(2.0 ** 120)]
    for g in scales:
        check(boundary_walk(g), g)


def test_special_values():
    check(np.array([0.0, -0.0, np.nan, -np.nan, 1e-45, -1e-45, 127 * 0.01, -127 * 0.01], f32), f32(0.01))
    step = f32(2.0 ** -149)  # subnormal scale: the row divides per element
    check(np.array([190 * step, step, 0, -3 * step], f32), step)
    check(np.array([1.0, -1.0, 0.0], f32), f32(np.inf))  # amax = inf
    check(np.array([1.0, -1.0, 0.0], f32), f32(0.0))  # all-zero row: gamma 0


def kernel_gamma(amax):
    """nlg_gamma_of: RN(amax / 127) by the same correction step with the
    constant y = RN(1/127); amax below 2^-90 (or not finite) divides."""
    amax = np.asarray(amax, f32)
    y = (f32(1.0) / f32(127.0)).astype(f32)
    with np.errstate(all="ignore"):
        q0 = (amax * y).astype(f32)
        fast = fmaf(fmaf(-q0, f32(127.0), amax), y, q0)
        slow = (amax / f32(127.0)).astype(f32)
    return np.where((amax >= FAST_MIN) & np.isfinite(amax), fast, slow)


def test_gamma_is_the_ieee_division():
    """Every significand at two exponents, and random values at every
    exponent from 2^-149 to 2^127, against float32 amax / 127."""
    sig = np.arange(1 << 23, dtype=np.uint32)
    for e in (127, 127 + 60):  # amax in [1, 2) and [2^60, 2^61)
        amax = ((np.uint32(e) << 23) | sig).view(f32)
        with np.errstate(all="ignore"):
            assert np.array_equal(kernel_gamma(amax), (amax / f32(127.0)).astype(f32))
    rng = np.random.default_rng(5)
    bits = rng.integers(0, 0x7F800000, 4_000_000, dtype=np.uint32)  # every finite positive float
    amax = bits.view(f32)
    with np.errstate(all="ignore"):
        assert np.array_equal(kernel_gamma(amax), (amax / f32(127.0)).astype(f32))


def test_without_the_correction_step_bytes_flip():
    """The check has teeth: q0 = RN(v*y) alone (no correction) misrounds
    some quotient next to a boundary, and that flips bytes."""
    rng = np.random.default_rng(11)
    flips = 0
    for _ in range(20):
        g = f32(f32(10.0 ** rng.uniform(-10, 10)) * f32(rng.uniform(1, 2)))
        v = boundary_walk(g, ulps=6)
        flips += int((kernel_byte(v, g, correct=False) != reference_byte(v, g)).sum())
    assert flips > 0
