"""Seeded test cases for every kernel name, in the reference's buffer layouts
(lisp/nelisp-gpu-kernels.el :buffers order, uint32 push constants).

Each case lists its buffers as 4-byte numpy arrays (float32 or uint32), the
push constants and the workgroup count a reference caller would pass
(ceil(domain/64), e.g. test/ternary-kernel-test.el:100), the index of a
buffer that is the same binding as an earlier one (in-place kernels), and the
parity bar: EXACT (bitwise) or a relative tolerance against the largest
reference magnitude, or ELEM(tol) for a per-element relative bound.
"""
from __future__ import annotations

import math
import struct
from dataclasses import dataclass, field

import numpy as np

EXACT = "exact"


@dataclass
class ELEM:
    tol: float


@dataclass
class Case:
    name: str
    bufs: list
    push: list
    groups: int
    tol: object = EXACT
    alias: dict = field(default_factory=dict)  # buffer index -> earlier index it aliases
    label: str = ""


def g64(n):
    return max(1, (int(n) + 63) // 64)


def f32bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def _f(rng, n, s=1.0):
    return (rng.standard_normal(n) * s).astype(np.float32)


def _z(n):
    return np.zeros(int(n), dtype=np.float32)


def _u32_as_f32(u):
    return np.asarray(u, dtype=np.uint32).view(np.float32).copy()


def cases(seed: int = 1234) -> list[Case]:
    rng = np.random.default_rng(seed)
    cs: list[Case] = []
    n = 1000
    for nm in ("vadd", "add2", "mul"):
        cs.append(Case(nm, [_f(rng, n), _f(rng, n), _z(n)], [n], g64(n)))
    cs.append(Case("scale", [_f(rng, n), np.array([0.3], np.float32), _z(n)], [n], g64(n)))
    Nn = 37
    cs.append(Case("causal-mask", [_f(rng, Nn * Nn)], [Nn], g64(Nn * Nn)))
    cs.append(Case("silu", [_f(rng, n, 4), _z(n)], [n], g64(n), 1e-6))
    cs.append(Case("silu-mul", [_f(rng, n, 4), _f(rng, n), _z(n)], [n], g64(n), 1e-6))
    M, N = 5, 300
    cs.append(Case("rmsnorm-fwd", [_f(rng, M * N), np.abs(_f(rng, M)) + 0.1, _f(rng, N), _z(M * N)],
                   [M, N], g64(M * N)))
    M, N = 7, 2560
    cs.append(Case("rmsnorm-istd", [_f(rng, M * N), _z(M)], [M, N], g64(M), 1e-5))
    seq, nh, hd = 3, 4, 128
    cs.append(Case("rmsnorm-heads", [_f(rng, seq * nh * hd), _f(rng, hd), _z(seq * nh * hd)],
                   [seq, nh, hd], g64(seq * nh), 1e-5))
    for (M, N) in ((40, 1000), (16, 4096), (3, 9000)):
        a = _f(rng, M * N, 3)
        a[::7] = -1.0e30
        cs.append(Case("softmax", [a, _z(M * N)], [M, N], g64(M), ELEM(1e-5), label=f"{M}x{N}"))
    a = _f(rng, 8 * 512, 3)
    a[5::11] = -np.inf
    cs.append(Case("softmax", [a, a], [8, 512], 1, ELEM(1e-5), alias={1: 0}, label="in-place"))
    seq, dim, vocab = 6, 64, 50
    tok = np.array([3, 0, 49, 7, vocab + 3, 12], np.float32)  # one id past the table
    cs.append(Case("embed-gather", [tok, _f(rng, vocab * dim), _z(seq * dim)], [seq, dim], g64(seq * dim)))
    kvdim = 96
    cs.append(Case("cache-append", [_f(rng, kvdim), np.array([5.0], np.float32), _f(rng, 8 * kvdim)],
                   [kvdim], g64(kvdim)))
    B, kvd, maxseq = 3, 32, 8
    cs.append(Case("cache-append-b", [_f(rng, B * kvd), np.array([3.0], np.float32),
                                      _f(rng, B * maxseq * kvd)], [B, kvd, maxseq], g64(B * kvd)))
    dim, kvd, wbase = 64, 16, 32
    cs.append(Case("qkv-append", [_f(rng, dim + 2 * kvd), _f(rng, 64), _f(rng, 64)], [dim, kvd, wbase],
                   g64(kvd)))

    def tables(rows, half, base=10000.0):
        p = np.arange(rows)[:, None]
        m = np.arange(half)[None, :]
        th = p / base ** (2.0 * m / (2 * half))
        return np.cos(th).astype(np.float32).ravel(), np.sin(th).astype(np.float32).ravel()

    cols, heads = 256, 2
    co, si = tables(16, 64)
    cs.append(Case("decode-rope", [_f(rng, cols), co, si, np.array([1.0], np.float32),
                                   np.array([7.0], np.float32), _z(cols)], [cols, heads], g64(heads * 64)))
    B, cols, heads = 3, 192, 3  # hd 64
    co, si = tables(16, 32)
    cs.append(Case("decode-rope-b", [_f(rng, B * cols), co, si, np.array([1.0], np.float32),
                                     np.array([11.0], np.float32), _z(B * cols)], [B, cols, heads],
                   g64(B * heads * 32)))
    seq, dim, heads = 5, 64, 4  # hd 16
    co, si = tables(seq, 8)
    cs.append(Case("rope-apply", [_f(rng, seq * dim), co, si, np.array([-1.0], np.float32), _z(seq * dim)],
                   [seq, dim, heads], g64(seq * heads * 8)))
    seq, nh, hd = 5, 3, 64
    cs.append(Case("rope-half", [_f(rng, seq * nh * hd), _z(seq * nh * hd)],
                   [seq, nh, hd, f32bits(10000.0), f32bits(1.0)], g64(seq * nh * 32), 1e-5))
    seq, cols = 5, 1001
    x = _f(rng, seq * cols, 2)
    x[3 * cols: 4 * cols] = 0.0  # an all-zero row: gamma 0, zero lanes
    for ng in ((cols + 3) // 4, (cols + 3) // 4 + 9):
        cs.append(Case("pack-act-rows", [x, _z(seq * ng), _z(seq)], [seq, cols, ng], g64(seq),
                       label=f"ng={ng}"))
    seq, cols = 5, 300
    cs.append(Case("quant-act", [_f(rng, seq * cols, 2), _z(seq * cols)], [seq, cols], g64(seq)))
    nn = 300
    cs.append(Case("dp4a-dot", [rng.integers(0, 65536, nn).astype(np.float32) for _ in range(4)] + [_z(nn)],
                   [nn], g64(nn)))
    seq, out, ng = 3, 40, 50
    halves = [rng.integers(0, 65536, k).astype(np.float32) for k in (seq * ng, seq * ng, out * ng, out * ng)]
    cs.append(Case("bitlinear-dp4a", halves + [_f(rng, out), np.array([0.02], np.float32),
                                              np.abs(_f(rng, seq)), _z(seq * out)], [seq, out, ng],
                   g64(seq * out)))
    for nm, nbeta in (("bitlinear-dp4a-1f", 1), ("bitlinear-dp4a-rows", out)):
        ap = _u32_as_f32(rng.integers(0, 2 ** 32, seq * ng, dtype=np.uint64))
        wp = _u32_as_f32(rng.integers(0, 2 ** 32, out * ng, dtype=np.uint64))
        cs.append(Case(nm, [ap, wp, _f(rng, out), np.abs(_f(rng, nbeta)) * 0.05, np.abs(_f(rng, seq)),
                            _z(seq * out)], [seq, out, ng], g64(seq * out)))
    for (seq, out, cols, nblk) in ((3, 6, 256, 2), (2, 9, 300, 3), (1, 5, 300, 1)):
        wng = (cols + 15) // 16
        w = _u32_as_f32(rng.integers(0, 2 ** 32, out * wng, dtype=np.uint64))
        cs.append(Case("ternary-rows", [_f(rng, seq * cols), w, _f(rng, out), np.abs(_f(rng, out * nblk)) * 0.05,
                                        _z(seq * out)], [seq, out, cols, nblk, wng], g64(seq * out), 1e-5,
                       label=f"{seq}x{out}x{cols}/{nblk}"))
    seq, inn, out, pk = 3, 100, 20, 12
    fcount = (inn + pk - 1) // pk
    codes = rng.integers(0, 3, (out, fcount, pk))
    wpk = (codes * (4 ** np.arange(pk))).sum(axis=2).astype(np.float32).ravel()
    for nm, nbeta in (("bitlinear-packed", 1), ("bitlinear-packed-v", out)):
        cs.append(Case(nm, [_f(rng, seq * inn), wpk, _f(rng, out), np.abs(_f(rng, nbeta)) * 0.1,
                            _z(seq * out)], [seq, inn, out, pk, fcount], g64(seq * out), 1e-5))
    # The f32 GEMMs sum in the reference's order (serial k; matmul-tiled's
    # right-nested 16-term tile sums), so they are bit-exact.  K = 300 and
    # 520 cross the device's 256-deep LDS stages; the 256^3 case is config 1.
    # Fewer groups than the domain needs: only the covered outputs change.
    for (M, K, N) in ((20, 24, 12), (64, 80, 72), (36, 300, 20), (256, 256, 256), (16, 520, 32)):
        A, Bm = _f(rng, M * K), _f(rng, K * N)
        C0 = _f(rng, M * N)
        lab = f"{M}x{K}x{N}"
        cs.append(Case("matmul", [A, Bm, _z(M * N)], [M, K, N], g64(M * N), label=lab))
        cs.append(Case("matmul", [A, Bm, C0], [M, K, N], max(1, g64(M * N) // 3), label=lab + "/partial"))
        tiles = ((M + 15) // 16) * ((N + 15) // 16)
        cs.append(Case("matmul-tiled", [A, Bm, _z(M * N)], [M, K, N], tiles, label=lab))
        cs.append(Case("matmul-tiled", [A, Bm, C0], [M, K, N], max(1, tiles - 2), label=lab + "/partial"))
        if M % 4 == 0 and N % 4 == 0:
            blocks = (M // 4) * (N // 4)
            cs.append(Case("matmul-reg", [A, Bm, _z(M * N)], [M, K, N], g64(blocks), label=lab))
            if blocks > 64:
                cs.append(Case("matmul-reg", [A, Bm, C0], [M, K, N], g64(blocks) - 1, label=lab + "/partial"))
    for (M, IN, OUT) in ((20, 12, 16), (9, 300, 70)):
        X, W, Bv = _f(rng, M * IN), _f(rng, OUT * IN), _f(rng, OUT)
        cs.append(Case("linear", [X, W, Bv, _z(M * OUT)], [M, IN, OUT], g64(M * OUT), label=f"{M}x{IN}x{OUT}"))
        cs.append(Case("linear", [X, W, Bv, _f(rng, M * OUT)], [M, IN, OUT], max(1, g64(M * OUT) // 2),
                       label=f"{M}x{IN}x{OUT}/partial"))
    seq, dim, heads, kvh = 9, 64, 4, 2
    cs.append(Case("attn-scores", [_f(rng, seq * dim), _f(rng, seq * kvh * 16), _z(heads * seq * seq)],
                   [seq, dim, heads, kvh], g64(heads * seq * seq)))
    cs.append(Case("attn-context", [np.abs(_f(rng, heads * seq * seq)), _f(rng, seq * kvh * 16), _z(seq * dim)],
                   [seq, dim, heads, kvh], g64(seq * dim)))
    dim, heads, kvh, maxseq = 256, 2, 1, 16
    cs.append(Case("decode-attn", [_f(rng, dim), _f(rng, maxseq * kvh * 128), _f(rng, maxseq * kvh * 128),
                                   np.array([9.0], np.float32), _z(dim)], [dim, heads, kvh], g64(dim), 1e-5))
    B, dim, heads, kvh, maxseq = 3, 256, 4, 2, 12
    cs.append(Case("decode-attn-b", [_f(rng, B * dim), _f(rng, B * maxseq * kvh * 64),
                                     _f(rng, B * maxseq * kvh * 64), np.array([5.0], np.float32),
                                     _z(B * dim)], [B, dim, heads, kvh, maxseq], g64(B * dim), 1e-5))
    seq, heads, kvh, hd = 17, 4, 2, 32
    cs.append(Case("attn-causal-gqa", [_f(rng, seq * heads * hd), _f(rng, seq * kvh * hd),
                                       _f(rng, seq * kvh * hd), _z(seq * heads * hd)], [seq, heads, kvh, hd],
                   g64(heads * seq), 1e-5))
    # transposed linears: X = W^T (BETA * G), seq positions at once
    for (out, cols, nblk, seq) in ((40, 300, 3, 2), (7, 256, 2, 1)):
        wng = (cols + 15) // 16
        w = _u32_as_f32(rng.integers(0, 2 ** 32, out * wng, dtype=np.uint64))
        cs.append(Case("ternary-rows-t", [w, np.abs(_f(rng, out * nblk)) * 0.05, _f(rng, seq * out),
                                          _z(seq * cols)], [out, cols, nblk, wng, seq], g64(seq * cols), 1e-5,
                       label=f"{out}x{cols}x{seq}"))
    out, cols, seq = 40, 150, 3
    ng = (cols + 3) // 4
    w = _u32_as_f32(rng.integers(0, 2 ** 32, out * ng, dtype=np.uint64))
    cs.append(Case("dp4a-rows-t", [w, np.abs(_f(rng, out)) * 0.05, _f(rng, seq * out), _z(seq * cols)],
                   [out, cols, ng, seq], g64(seq * cols), 1e-5))
    # long-context decode: StreamingLLM ring (nsink 2 + win 6 slots) and a
    # paged pool (blocks of 4 positions, 5 blocks per sequence)
    kvd, nsink, win = 32, 2, 6
    for pos in (4.0, 13.0):  # inside the first window; wrapped around it
        cs.append(Case("cache-append-ring", [_f(rng, kvd), np.array([pos], np.float32),
                                            _f(rng, (nsink + win) * kvd)], [kvd, nsink, win], g64(kvd),
                       label=f"pos={int(pos)}"))
    dim, heads, kvh = 256, 4, 2  # hd 64
    co, si = tables(32, 32)
    for pos in (5.0, 20.0):  # before and after the window fills
        cs.append(Case("decode-attn-stream", [_f(rng, dim), _f(rng, (nsink + win) * kvh * 64),
                                             _f(rng, (nsink + win) * kvh * 64), np.array([pos], np.float32), co,
                                             si, _z(dim)], [dim, heads, kvh, nsink, win], g64(dim), 1e-5,
                       label=f"pos={int(pos)}"))
    ne, qcrel = 7, 9
    ent = np.array([[(r * 3 % 10) * kvh * 64, r + 2] for r in range(ne)], np.float32).ravel()
    cs.append(Case("attn-stream-entries", [_f(rng, dim), _f(rng, 10 * kvh * 64), _f(rng, 10 * kvh * 64), ent, co,
                                          si, _z(dim)], [dim, heads, kvh, ne, qcrel], g64(dim), 1e-5))
    B, kvd, bs, mbps, nblk = 3, 32, 4, 5, 16
    table = rng.permutation(nblk)[:B * mbps].astype(np.float32)
    cs.append(Case("cache-append-paged", [_f(rng, B * kvd), np.array([9.0], np.float32), table,
                                         _f(rng, nblk * bs * kvd)], [B, kvd, bs, mbps], g64(B * kvd)))
    lens = np.array([3.0, 17.0, 10.0], np.float32)
    cs.append(Case("cache-append-paged-v", [_f(rng, B * kvd), lens, table, _f(rng, nblk * bs * kvd)],
                   [B, kvd, bs, mbps], g64(B * kvd)))
    B, dim, heads, kvh = 3, 256, 4, 2  # hd 64, kvdim 128
    pool = nblk * bs * kvh * 64
    cs.append(Case("decode-attn-paged", [_f(rng, B * dim), _f(rng, pool), _f(rng, pool), np.array([13.0], np.float32),
                                        table, _z(B * dim)], [B, dim, heads, kvh, bs, mbps], g64(B * dim), 1e-5))
    cs.append(Case("decode-attn-paged-v", [_f(rng, B * dim), _f(rng, pool), _f(rng, pool), lens, table,
                                          _z(B * dim)], [B, dim, heads, kvh, bs, mbps], g64(B * dim), 1e-5))
    cs.append(Case("block-copy", [_f(rng, nblk * bs * kvd)], [bs, kvd, 3, 11], g64(bs * kvd)))
    B, cols, heads = 3, 192, 3  # hd 64
    co, si = tables(24, 32)
    cs.append(Case("decode-rope-b-v", [_f(rng, B * cols), co, si, np.array([1.0], np.float32),
                                       np.array([2.0, 17.0, 9.0], np.float32), _z(B * cols)], [B, cols, heads],
                   g64(B * heads * 32)))
    return cs


def case_id(c: Case) -> str:
    return c.name + (f"[{c.label}]" if c.label else "")
