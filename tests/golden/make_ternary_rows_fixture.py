"""Write tests/golden/ternary_rows_lcg.npz: the inputs and expected outputs
of the reference's own ternary-kernel test, regenerated from its generator.

test/ternary-kernel-test.el draws everything from one LCG,
seed <- (seed*1103515245 + 12345) mod 2^31, starting at 20260921 (:17,
:36-38), in this order (:60-66): per output row o, the bias (0.4r - 0.2),
then nblk block scales (0.01 + 0.05r), then cols trits (floor(3r) - 1);
then x (2r - 1) and g (2r - 1).  Shapes seq=3, out=6, cols=256, bsize=128
(:53-54).  The expected forward output is the test's scalar CPU sum in
double precision (tk-cpu-forward, :79-89): y = bias + sum_i trit*beta*x.
Elisp floats are IEEE doubles, so this restates that arithmetic exactly.
The trits are packed with the test's tk-pack layout (:40-50).

Run:  python tests/golden/make_ternary_rows_fixture.py
"""
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def lcg_stream(seed: int):
    while True:
        seed = (seed * 1103515245 + 12345) % 2147483648
        yield seed / 2147483648.0


def build():
    seq, out, cols, bsize = 3, 6, 256, 128
    nblk, wng = cols // bsize, cols // 16
    r = lcg_stream(20260921)
    bias = np.zeros(out)
    beta = np.zeros(out * nblk)
    trits = np.zeros((out, cols), dtype=np.int64)
    for o in range(out):
        bias[o] = 0.4 * next(r) - 0.2
        for b in range(nblk):
            beta[o * nblk + b] = 0.01 + 0.05 * next(r)
        for i in range(cols):
            trits[o, i] = int(3.0 * next(r)) - 1  # (truncate (* 3.0 r)) - 1
    x = np.array([2.0 * next(r) - 1.0 for _ in range(seq * cols)])
    g = np.array([2.0 * next(r) - 1.0 for _ in range(seq * out)])
    # tk-pack: field i of row o in byte o*wng*4 + i>>2 at shift 2*(i&3)
    packed = bytearray(out * wng * 4)
    for o in range(out):
        for i in range(cols):
            v = trits[o, i]
            code = 1 if v == 1 else (3 if v == -1 else 0)
            idx = o * wng * 4 + (i >> 2)
            packed[idx] |= code << (2 * (i & 3))
    wp = np.frombuffer(bytes(packed), dtype="<u4").copy()
    # tk-cpu-forward, in double, serial in i as the Elisp loop
    y = np.zeros(seq * out)
    for s in range(seq):
        for o in range(out):
            acc = 0.0
            for i in range(cols):
                acc = acc + trits[o, i] * beta[o * nblk + i // bsize] * x[s * cols + i]
            y[s * out + o] = bias[o] + acc
    return dict(seq=seq, out=out, cols=cols, nblk=nblk, wng=wng, bias=bias, beta=beta,
                trits=trits.astype(np.int8), x=x, g=g, wp=wp, y=y)


if __name__ == "__main__":
    d = build()
    np.savez(os.path.join(HERE, "ternary_rows_lcg.npz"), **d)
    print("wrote ternary_rows_lcg.npz", {k: np.shape(v) for k, v in d.items()})
