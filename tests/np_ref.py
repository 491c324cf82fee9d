"""Independent numpy statements of each kernel's mathematics, used to pin the
C restatement (oracle/nlg_oracle.c) on the CPU.

Float kernels are stated as closed forms in float64 (softmax =
exp(x - max)/sum, attention = softmax(q.k/sqrt(hd)).V, RMSNorm, rotations by
angle, matrix products) and compared within a tolerance.  Kernels whose
reference output is a fixed sequence of single f32 operations (copies,
gathers, adds, table rotations, quantisation) are stated with vectorised
float32 numpy ops -- indexing written from the layouts, not from the loop
bodies -- and compared bitwise.  Integer kernels are brute-forced in int64.
"""
from __future__ import annotations

import numpy as np

import nlgpu


def _i8(words):
    """uint32 words -> [n, 4] signed int8 lanes (lane l = byte l)."""
    return np.asarray(words, dtype=np.uint32).view(np.int8).reshape(-1, 4).astype(np.int64)


def u16pair(lo, hi):
    return (lo.astype(np.uint64) + hi.astype(np.uint64) * 65536).astype(np.uint32)


def ref(case):
    """Expected output buffers {index: array} for a kernel_specs.Case."""
    b = [np.array(x, copy=True) for x in case.bufs]
    p = case.push
    nm = case.name
    f32 = np.float32
    if nm in ("vadd", "add2"):
        return {2: (b[0] + b[1]).astype(f32)}
    if nm == "mul":
        return {2: (b[0] * b[1]).astype(f32)}
    if nm == "scale":
        return {2: (b[0] * b[1][0]).astype(f32)}
    if nm == "causal-mask":
        Nn = p[0]
        s = b[0].reshape(Nn, Nn).copy()
        s[np.triu_indices(Nn, 1)] = f32(-1.0e30)
        return {0: s.ravel()}
    if nm == "silu":
        x = b[0].astype(np.float64)
        return {1: x / (1.0 + np.exp(-x))}
    if nm == "silu-mul":
        x = b[0].astype(np.float64)
        return {2: x / (1.0 + np.exp(-x)) * b[1]}
    if nm == "rmsnorm-fwd":
        M, N = p
        return {3: ((b[0].reshape(M, N) * b[1][:, None]) * b[2][None, :]).astype(f32).ravel()}
    if nm == "rmsnorm-istd":
        M, N = p
        x = b[0].reshape(M, N).astype(np.float64)
        return {1: 1.0 / np.sqrt((x * x).mean(axis=1) + 1e-6)}
    if nm == "rmsnorm-heads":
        seq, nh, hd = p
        x = b[0].reshape(seq * nh, hd).astype(np.float64)
        inv = 1.0 / np.sqrt((x * x).mean(axis=1) + 1e-6)
        return {2: (x * inv[:, None] * b[1][None, :]).ravel()}
    if nm == "softmax":
        M, N = p
        x = b[0].reshape(M, N).astype(np.float64)
        e = np.exp(x - x.max(axis=1, keepdims=True))
        return {1: (e / e.sum(axis=1, keepdims=True)).ravel()}
    if nm == "embed-gather":
        seq, dim = p
        tab = b[1].reshape(-1, dim)
        tok = b[0].astype(np.int64)
        outp = np.zeros((seq, dim), f32)
        ok = tok < tab.shape[0]
        outp[ok] = tab[tok[ok]]
        return {2: outp.ravel()}
    if nm == "cache-append":
        kvdim = p[0]
        pos = int(b[1][0])
        c = b[2].copy()
        c[pos * kvdim:(pos + 1) * kvdim] = b[0]
        return {2: c}
    if nm == "cache-append-b":
        B, kvdim, maxseq = p
        pos = int(b[1][0])
        c = b[2].reshape(B, maxseq, kvdim).copy()
        c[:, pos, :] = b[0].reshape(B, kvdim)
        return {2: c.ravel()}
    if nm == "qkv-append":
        dim, kvdim, wbase = p
        ck, cv = b[1].copy(), b[2].copy()
        ck[wbase:wbase + kvdim] = b[0][dim:dim + kvdim]
        cv[wbase:wbase + kvdim] = b[0][dim + kvdim:dim + 2 * kvdim]
        return {1: ck, 2: cv}
    if nm in ("decode-rope", "decode-rope-b", "decode-rope-b-v", "rope-apply"):
        if nm == "decode-rope-b-v":
            B, cols, heads = p
            rows, dim = B, cols
            pos = b[4][:B].astype(np.int64)
        elif nm == "decode-rope":
            cols, heads = p
            rows, pos = 1, np.array([int(b[4][0])])
            dim = cols
        elif nm == "decode-rope-b":
            B, cols, heads = p
            rows, dim = B, cols
            pos = np.full(B, int(b[4][0]))
        else:
            seq, dim, heads = p
            rows = seq
            pos = np.arange(seq)
        hd = dim // heads
        half = hd // 2
        x = b[0].reshape(rows, heads, half, 2)
        co = b[1].reshape(-1, half)[pos][:, None, :]
        si = (b[2].reshape(-1, half)[pos] * b[3][0]).astype(f32)[:, None, :]
        a0, a1 = x[..., 0], x[..., 1]
        y = np.stack([(a0 * co) - (a1 * si), (a0 * si) + (a1 * co)], axis=-1).astype(f32)
        out_idx = 5 if nm != "rope-apply" else 4
        return {out_idx: y.ravel()}
    if nm == "rope-half":
        seq, nh, hd = p[:3]
        rbase = np.frombuffer(np.uint32(p[3]).tobytes(), f32)[0]
        sgn = np.frombuffer(np.uint32(p[4]).tobytes(), f32)[0]
        half = hd // 2
        x = b[0].reshape(seq, nh, hd).astype(np.float64)
        pos = np.arange(seq)[:, None, None]
        m = np.arange(half)[None, None, :]
        th = pos / float(rbase) ** (2.0 * m / hd)
        c, s = np.cos(th), sgn * np.sin(th)
        a0, a1 = x[..., :half], x[..., half:]
        return {1: np.concatenate([a0 * c - a1 * s, a1 * c + a0 * s], axis=-1).ravel()}
    if nm == "pack-act-rows":
        seq, cols, ng = p
        x = b[0].reshape(seq, cols)
        amax = np.max(np.abs(x), axis=1).astype(f32)
        gamma = (amax / f32(127.0)).astype(f32)
        with np.errstate(divide="ignore", invalid="ignore"):
            q = np.where(gamma[:, None] > 0, x / gamma[:, None], f32(0)).astype(f32)
        r = np.minimum(np.trunc((np.abs(q) + f32(0.5)).astype(f32)), 127).astype(np.int64)
        lanes = np.where(q < 0, (256 - r) % 256, r).astype(np.uint32)
        full = np.zeros((seq, ng * 4), np.uint32)
        w = min(cols, ng * 4)
        full[:, :w] = lanes[:, :w]
        words = (full.reshape(seq, ng, 4) << (8 * np.arange(4, dtype=np.uint32))).sum(axis=2).astype(np.uint32)
        return {1: words.ravel().view(f32), 2: gamma}
    if nm == "quant-act":
        seq, cols = p
        x = b[0].reshape(seq, cols)
        gamma = (np.max(np.abs(x), axis=1).astype(f32) / f32(127.0)).astype(f32)[:, None]
        with np.errstate(divide="ignore", invalid="ignore"):
            q = np.where(gamma > 0, x / gamma, f32(0)).astype(f32)
        rf = np.minimum(np.trunc((np.abs(q) + f32(0.5)).astype(f32)), f32(127)).astype(f32)
        sgn = np.where(q < 0, f32(-1.0), f32(1.0)).astype(f32)
        xq = np.where(gamma > 0, gamma * (sgn * rf), f32(0)).astype(f32)
        return {1: xq.ravel()}
    if nm == "dp4a-dot":
        a = u16pair(b[0], b[1])
        c = u16pair(b[2], b[3])
        return {4: (_i8(a) * _i8(c)).sum(axis=1).astype(f32)}
    if nm in ("bitlinear-dp4a", "bitlinear-dp4a-1f", "bitlinear-dp4a-rows"):
        seq, out, ng = p
        if nm == "bitlinear-dp4a":
            ap, wp = u16pair(b[0], b[1]), u16pair(b[2], b[3])
            bias, beta, gamma, yi = b[4], b[5], b[6], 7
        else:
            ap, wp = b[0].view(np.uint32), b[1].view(np.uint32)
            bias, beta, gamma, yi = b[2], b[3], b[4], 5
        A = _i8(ap).reshape(seq, ng * 4)
        W = _i8(wp).reshape(out, ng * 4)
        acc = (A @ W.T).astype(np.int64)
        acc = ((acc + 2 ** 31) % 2 ** 32 - 2 ** 31).astype(f32)
        be = beta[:out] if nm == "bitlinear-dp4a-rows" else np.full(out, beta[0], f32)
        y = bias[None, :] + ((be[None, :] * gamma[:, None]).astype(f32) * acc).astype(f32)
        return {yi: y.astype(f32).ravel()}
    if nm == "ternary-rows":
        seq, out, cols, nblk, wng = p
        wq = nlgpu.unpack_ternary(b[1].view(np.uint32).reshape(out, wng), cols).astype(np.float64)
        nw = min(wng, 8 * nblk)
        wq[:, nw * 16:] = 0.0  # words the reference's block loop never visits
        blk = np.arange(cols) // 128
        beta = b[3].reshape(out, nblk).astype(np.float64)
        bb = np.where(blk[None, :] < nblk, beta[:, np.minimum(blk, nblk - 1)], 0.0)
        x = b[0].reshape(seq, cols).astype(np.float64)
        return {4: (b[2][None, :] + x @ (wq * bb).T).ravel()}
    if nm in ("bitlinear-packed", "bitlinear-packed-v"):
        seq, inn, out, pk, fcount = p
        packed = b[1].reshape(out, fcount).astype(np.int64)
        codes = (packed[:, :, None] // (4 ** np.arange(pk))[None, None, :]) % 4
        tern = (codes.reshape(out, fcount * pk)[:, :inn] - 1).astype(np.float64)
        be = b[3][:out] if nm.endswith("-v") else np.full(out, b[3][0])
        x = b[0].reshape(seq, inn).astype(np.float64)
        return {4: (b[2][None, :] + (x @ tern.T) * be[None, :]).ravel()}
    if nm in ("matmul", "matmul-tiled", "matmul-reg", "linear"):
        if nm == "linear":
            M, IN, N = p
            full = b[0].reshape(M, IN).astype(np.float64) @ b[1].reshape(N, IN).T + b[2]
            cidx = 3
        else:
            M, K, N = p
            full = b[0].reshape(M, K).astype(np.float64) @ b[1].reshape(K, N)
            cidx = 2
        # a partial grid writes only the outputs of the invocations it runs
        r, c = np.meshgrid(np.arange(M), np.arange(N), indexing="ij")
        if nm == "matmul-tiled":
            covered = (r // 16) * ((N + 15) // 16) + c // 16 < case.groups  # workgroup = tile
        elif nm == "matmul-reg":
            covered = (r // 4) * ((N + 3) // 4) + c // 4 < 64 * case.groups  # invocation = 4x4 block
        else:
            covered = r * N + c < 64 * case.groups  # invocation = output
        return {cidx: np.where(covered, full, b[cidx].reshape(M, N).astype(np.float64)).ravel()}
    if nm == "attn-scores":
        seq, dim, heads, kvh = p
        hd = dim // heads
        grp = heads // kvh
        q = b[0].reshape(seq, heads, hd).astype(np.float64)
        k = b[1].reshape(seq, kvh, hd).astype(np.float64)
        s = np.einsum("ihd,jhd->hij", q, np.repeat(k, grp, axis=1)) / np.sqrt(hd)
        s[:, np.triu_indices(seq, 1)[0], np.triu_indices(seq, 1)[1]] = -1.0e30
        return {2: s.ravel()}
    if nm == "attn-context":
        seq, dim, heads, kvh = p
        hd = dim // heads
        grp = heads // kvh
        P = b[0].reshape(heads, seq, seq).astype(np.float64)
        v = np.repeat(b[1].reshape(seq, kvh, hd).astype(np.float64), grp, axis=1)
        return {2: np.einsum("hij,jhd->ihd", P, v).ravel()}
    if nm in ("decode-attn", "decode-attn-b"):
        if nm == "decode-attn":
            dim, heads, kvh = p
            B, maxseq = 1, 0
        else:
            B, dim, heads, kvh, maxseq = p
        hd = dim // heads
        grp = heads // kvh
        L = int(b[3][0]) + 1
        ms = maxseq if B > 1 or maxseq else L
        q = b[0].reshape(B, heads, hd).astype(np.float64)
        ck = b[1].reshape(B, -1, kvh, hd)[:, :L].astype(np.float64) if maxseq else b[1].reshape(1, -1, kvh, hd)[:, :L].astype(np.float64)
        cv = b[2].reshape(B, -1, kvh, hd)[:, :L].astype(np.float64) if maxseq else b[2].reshape(1, -1, kvh, hd)[:, :L].astype(np.float64)
        ck = np.repeat(ck, grp, axis=2)
        cv = np.repeat(cv, grp, axis=2)
        s = np.einsum("bhd,bjhd->bhj", q, ck) / np.sqrt(hd)
        e = np.exp(s - s.max(axis=2, keepdims=True))
        w = e / e.sum(axis=2, keepdims=True)
        del ms
        return {4: np.einsum("bhj,bjhd->bhd", w, cv).ravel()}
    if nm in ("ternary-rows-t", "dp4a-rows-t"):
        if nm == "ternary-rows-t":
            out, cols, nblk, wng, seq = p
            w = np.asarray(b[0], f32).view(np.uint32)[:out * wng].reshape(out, wng)
            f = np.arange(cols)
            fields = ((w[:, f // 16] >> (2 * (f % 16)).astype(np.uint32)) & 3).astype(np.int64)
            wt = np.where(fields >= 2, fields - 4, fields).astype(np.float64)  # [out, cols]
            be = b[1][:out * nblk].reshape(out, nblk)[:, f // 128].astype(np.float64)
        else:
            out, cols, ng, seq = p
            wt = _i8(np.asarray(b[0], f32).view(np.uint32)[:out * ng]).reshape(out, ng * 4)[:, :cols]
            wt = wt.astype(np.float64)
            be = np.repeat(b[1][:out, None].astype(np.float64), cols, axis=1)
        g = b[2][:seq * out].reshape(seq, out).astype(np.float64)
        return {3: (g @ (wt * be)).ravel()}
    if nm == "cache-append-ring":
        kvdim, nsink, win = p
        pos = int(b[1][0])
        slot = pos if pos < nsink else nsink + (pos - nsink) % win
        c = b[2].copy()
        c[slot * kvdim:(slot + 1) * kvdim] = b[0][:kvdim]
        return {2: c}
    if nm in ("cache-append-paged", "cache-append-paged-v"):
        B, kvdim, bs, mbps = p
        pool = b[3].copy()
        for s_ in range(B):
            pos = int(b[1][s_ if nm.endswith("-v") else 0])
            phys = int(b[2][s_ * mbps + pos // bs])
            row = phys * bs + pos % bs
            pool[row * kvdim:(row + 1) * kvdim] = b[0][s_ * kvdim:(s_ + 1) * kvdim]
        return {3: pool}
    if nm == "block-copy":
        bs, kvdim, src, dst = p
        bn = bs * kvdim
        pool = b[0].copy()
        pool[dst * bn:(dst + 1) * bn] = b[0][src * bn:(src + 1) * bn]
        return {0: pool}
    if nm in ("decode-attn-stream", "attn-stream-entries"):
        dim, heads, kvh = p[:3]
        hd, grp = dim // heads, heads // kvh
        half, kvdim = hd // 2, kvh * hd
        if nm == "decode-attn-stream":
            nsink, win = p[3], p[4]
            pos, cap = int(b[3][0]), nsink + win
            n = min(pos + 1, cap)
            start = nsink if pos < cap else pos - win + 1
            woff = (start - nsink) % win
            slots = [r if r < nsink else nsink + (woff + r - nsink) % win for r in range(n)]
            rows = [(sl * kvdim, r) for r, sl in enumerate(slots)]
            qcrel = min(pos, cap - 1)
        else:
            ne, qcrel = p[3], p[4]
            rows = [(int(b[3][2 * r]), int(b[3][2 * r + 1])) for r in range(ne)]
        co = b[4].reshape(-1, half).astype(np.float64)
        si = b[5].reshape(-1, half).astype(np.float64)

        def rot(v, c):  # v [..., hd] pairs (2m, 2m+1) rotated by angle row c
            v0, v1 = v[..., 0:2 * half:2], v[..., 1:2 * half:2]
            return v0 * co[c] - v1 * si[c], v0 * si[c] + v1 * co[c]
        q = b[0].reshape(heads, hd).astype(np.float64)
        qr0, qr1 = rot(q, qcrel)
        outp = np.zeros((heads, hd))
        for h in range(heads):
            kvo = (h // grp) * hd
            sc = []
            for base, crel in rows:
                k = b[1][base + kvo: base + kvo + hd].astype(np.float64)
                k0, k1 = rot(k, crel)
                sc.append((qr0[h] * k0 + qr1[h] * k1).sum() / np.sqrt(hd))
            sc = np.array(sc)
            e = np.exp(sc - sc.max())
            vv = np.array([b[2][base + kvo: base + kvo + hd] for base, _ in rows], np.float64)
            outp[h] = (e[:, None] * vv).sum(axis=0) / e.sum()
        return {6: outp.ravel()}
    if nm in ("decode-attn-paged", "decode-attn-paged-v"):
        B, dim, heads, kvh, bs, mbps = p
        hd, grp = dim // heads, heads // kvh
        kvdim = kvh * hd
        outp = np.zeros((B, heads, hd))
        for s_ in range(B):
            n = int(b[3][s_ if nm.endswith("-v") else 0]) + 1
            rows = [(int(b[4][s_ * mbps + j // bs]) * bs + j % bs) * kvdim for j in range(n)]
            for h in range(heads):
                kvo = (h // grp) * hd
                q = b[0][s_ * dim + h * hd: s_ * dim + (h + 1) * hd].astype(np.float64)
                K = np.array([b[1][r + kvo: r + kvo + hd] for r in rows], np.float64)
                V = np.array([b[2][r + kvo: r + kvo + hd] for r in rows], np.float64)
                sc = K @ q / np.sqrt(hd)
                e = np.exp(sc - sc.max())
                outp[s_, h] = (e[:, None] * V).sum(axis=0) / e.sum()
        return {5: outp.ravel()}
    if nm == "attn-causal-gqa":
        seq, heads, kvh, hd = p
        grp = heads // kvh
        q = b[0].reshape(seq, heads, hd).astype(np.float64)
        k = np.repeat(b[1].reshape(seq, kvh, hd).astype(np.float64), grp, axis=1)
        v = np.repeat(b[2].reshape(seq, kvh, hd).astype(np.float64), grp, axis=1)
        s = np.einsum("ihd,jhd->hij", q, k) / np.sqrt(hd)
        s = np.where(np.tril(np.ones((seq, seq), bool))[None], s, -np.inf)
        e = np.exp(s - s.max(axis=2, keepdims=True))
        w = e / e.sum(axis=2, keepdims=True)
        return {3: np.einsum("hij,jhd->ihd", w, v).ravel()}
    raise KeyError(nm)


def compare(got: np.ndarray, want: np.ndarray, tol) -> tuple[bool, float]:
    """(ok, error) under a kernel_specs tolerance."""
    from kernel_specs import ELEM, EXACT
    g = np.asarray(got)
    w = np.asarray(want)
    if tol == EXACT:
        gb = g.astype(np.float32).view(np.uint32)
        wb = w.astype(np.float32).view(np.uint32)
        nbad = int(np.count_nonzero(gb != wb))
        return nbad == 0, float(nbad)
    g64 = g.astype(np.float64)
    w64 = w.astype(np.float64)
    if isinstance(tol, ELEM):
        fin = np.isfinite(w64)
        if not np.array_equal(np.isfinite(g64), fin):
            return False, float("inf")
        err = np.abs(g64[fin] - w64[fin]) / np.maximum(np.abs(w64[fin]), 1e-30)
        e = float(err.max()) if err.size else 0.0
        return e <= tol.tol, e
    scale = float(np.max(np.abs(w64))) if w64.size else 0.0
    e = float(np.max(np.abs(g64 - w64))) / max(scale, 1e-12) if w64.size else 0.0
    return e <= float(tol), e
