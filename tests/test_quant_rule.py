"""The division-free exact quantisation of the GPU kernels (lane_est /
quant_word in nelisp-gpu_amd/csrc/nlg_quant.h) against the reference's
rounding (pack-act-rows, lisp/nelisp-gpu-kernels.el:912-926:
ri = min(trunc(RN(RN(|v|/g) + 0.5)), 127)), both restated in numpy.

The kernels take t = RN(|v| * RN(1/g) + 0.5) (one fused multiply-add),
trust min(trunc(t), 127) when |frac(t) - 1/2| <= 1/2 - 2^-13 (t at least
2^-13 from an integer), and recompute every other element with the IEEE
division; a row whose 1/g is not finite (g = 0 or subnormal) divides
throughout.  The fused rounding is restated exactly: the product of two
float32 values is exact in float64, adding 0.5 to it is exact in float64
whenever the product is at least 2^-6, and below that t is within 2^-6 of
1/2, where a second rounding cannot move trunc(t) or the band test.  The
claim under test is that the trusted estimates are never wrong: checked on
random rows across 60 decades of scale and on values walked ulp by ulp across
every rounding boundary, where a guard band that is too narrow would show.
CPU only.
"""
import numpy as np

f32 = np.float32
BAND = f32(2.0 ** -13)


def exact_ri(v, g):
    with np.errstate(all="ignore"):
        q = (np.abs(v).astype(f32) / g).astype(f32)
        t = (q + f32(0.5)).astype(f32)
        return np.where(np.isnan(t), 0, np.minimum(np.trunc(np.nan_to_num(t, posinf=1e9)), 127)).astype(np.int64)


def kernel_ri(v, g):
    """The kernels' rule; returns (ri, fraction of elements sent to the exact path)."""
    with np.errstate(all="ignore"):
        ginv = (f32(1.0) / g).astype(f32)
        t = (np.abs(v).astype(np.float64) * np.float64(ginv) + 0.5).astype(f32)
        kf = np.trunc(t)
        fr = (t - kf).astype(f32)
        near = ~(np.abs((fr - f32(0.5)).astype(f32)) <= f32(0.5) - BAND)  # NaN lands here
        est = np.minimum(np.nan_to_num(kf), 127).astype(np.int64)
    if not (g > 0 and np.isfinite(ginv)):
        near = np.ones(v.shape, bool)
    return np.where(near, exact_ri(v, g), est), near.mean()


def check(v, g):
    v = np.asarray(v, f32)
    g = f32(g)
    want = exact_ri(v, g)
    got, frac = kernel_ri(v, g)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, (v[bad[:5]], got[bad[:5]], want[bad[:5]])
    return frac


def boundary_walk(g, ulps=8):
    centre = ((np.arange(1, 129, dtype=np.float64) - 0.5) * np.float64(g)).astype(f32)
    out, up, down = [centre], centre.copy(), centre.copy()
    for _ in range(ulps):
        up = np.nextafter(up, f32(np.inf))
        down = np.nextafter(down, f32(0))
        out += [up, down]
    v = np.concatenate(out)
    return np.concatenate([v, -v])


def test_random_rows():
    rng = np.random.default_rng(2024)
    for _ in range(20):
        amax = f32(10.0 ** rng.uniform(-30, 30))
        g = f32(amax / f32(127.0))
        v = (rng.uniform(-1, 1, 200_000) * amax).astype(f32)
        v[:2] = [amax, -amax]
        assert check(v, g) < 0.01  # the exact path stays rare


def test_every_rounding_boundary():
    rng = np.random.default_rng(7)
    scales = [f32(f32(10.0 ** rng.uniform(-20, 20)) * f32(rng.uniform(1, 2))) for _ in range(30)]
    scales += [f32(1.0), f32(2.0 ** -20), np.nextafter(f32(2.0), f32(0)), f32(2.0 ** -126), f32(2.0 ** -127)]
    for g in scales:
        check(boundary_walk(g), g)


def test_special_values():
    check(np.array([0.0, -0.0, np.nan, np.inf, -np.inf, 1e-45, -1e-45, 3e38], f32), f32(0.01))
    step = f32(2.0 ** -149)  # subnormal scale: the row divides throughout
    check(np.array([190 * step, step, 0, -3 * step], f32), step)
    check(np.array([1.0, -1.0, 0.0], f32), f32(np.inf))  # amax = inf
