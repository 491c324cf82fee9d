"""Pins of the CPU restatements the decoder-layer tests compare against
(CPU only): or_rmsnorm_rows against float64 RMSNorm, or_decode_attn_f16
against a float64 softmax-weighted sum over the fp16 caches, its fp16 decode
against numpy's for every one of the 65,536 bit patterns, the reference
RoPE's pos-0 identity, and the host generators the device stack mirrors."""
import numpy as np

import layer_ref as ref
import nlg_oracle as orc
import nlgpu

f32 = np.float32


def test_rmsnorm_rows_matches_float64():
    rng = np.random.default_rng(1)
    rows, cols = 5, 2560
    x = rng.standard_normal(rows * cols).astype(f32) * f32(3)
    g = rng.uniform(0.5, 1.5, cols).astype(f32)
    y = orc.rmsnorm_rows(x, g, 1e-5, rows, cols).reshape(rows, cols)
    xd = x.reshape(rows, cols).astype(np.float64)
    want = xd / np.sqrt((xd * xd).mean(axis=1, keepdims=True) + 1e-5) * g
    assert np.abs(y - want).max() <= 1e-5 * np.abs(want).max()
    # eps matters: an all-zero row stays zero, a tiny row is damped by eps
    z = orc.rmsnorm_rows(np.zeros(64, f32), np.ones(64, f32), 1e-5, 1, 64)
    assert np.all(z == 0)


def test_f16_decode_every_pattern():
    # pos 0: one position, e = exp(0) = 1, z = 1, so out = V row 0 exactly
    B, hd = 1024, 64
    v = np.arange(65536, dtype=np.uint16)
    k = np.zeros(65536, np.uint16)
    q = np.zeros(B * hd, f32)
    out = orc.decode_attn_f16(q, k, v, 0, B, 1, 1, hd, 1)
    want = v.view(np.float16).astype(f32)
    want = want + f32(0.0)  # ctx starts at +0.0, so a -0.0 row reads back +0.0
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(out), nan)
    assert np.array_equal(out[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_decode_attn_f16_matches_float64():
    rng = np.random.default_rng(2)
    B, heads, kvh, hd, max_seq, pos = 2, 8, 2, 64, 40, 33
    q = rng.standard_normal(B * heads * hd).astype(f32)
    kc = rng.standard_normal(B * kvh * max_seq * hd).astype(np.float16)
    vc = rng.standard_normal(B * kvh * max_seq * hd).astype(np.float16)
    out = orc.decode_attn_f16(q, kc.view(np.uint16), vc.view(np.uint16), pos, B, heads, kvh, hd, max_seq)
    K = kc.astype(np.float64).reshape(B, kvh, max_seq, hd)[:, :, :pos + 1]
    V = vc.astype(np.float64).reshape(B, kvh, max_seq, hd)[:, :, :pos + 1]
    Q = q.astype(np.float64).reshape(B, heads, hd)
    grp = heads // kvh
    want = np.empty((B, heads, hd))
    for b in range(B):
        for h in range(heads):
            s = K[b, h // grp] @ Q[b, h] / np.sqrt(hd)
            e = np.exp(s - s.max())
            want[b, h] = e @ V[b, h // grp] / e.sum()
    assert np.abs(out - want.ravel()).max() <= 1e-5 * np.abs(want).max()


def test_rope_at_position_zero_is_identity():
    x = np.random.default_rng(3).standard_normal(2 * 256).astype(f32)
    half = 32
    p = np.arange(4)[:, None] / (500000.0 ** (2.0 * np.arange(half)[None, :] / 64))
    co, si = np.cos(p).astype(f32).ravel(), np.sin(p).astype(f32).ravel()
    assert np.array_equal(ref.rope_b(x, co, si, 0, 2, 256, 4), x)
    y = ref.rope_b(x, co, si, 3, 2, 256, 4)
    # a rotation keeps each pair's length
    n0 = np.hypot(x[0::2].astype(np.float64), x[1::2])
    n1 = np.hypot(y[0::2].astype(np.float64), y[1::2])
    assert np.abs(n0 - n1).max() <= 1e-6 * n0.max()


def test_host_generators():
    z = nlgpu.normal_pairs(99, 200001)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01
    t = nlgpu.trits(5, (1000, 1000))
    assert abs((t == 0).mean() - 0.5) < 0.005 and abs((t == 1).mean() - 0.25) < 0.005
    assert nlgpu.stack_tensor_seed(7, 0, 3) == 7 + 1000003 + 3


class _HostStack:
    """Weights for the reference composition drawn on the host (the device
    stack's layout), so the composition can run without a GPU."""

    def __init__(self, seed=0, **cfg):
        class C:
            pass
        self.cfg = C()
        for k, v in cfg.items():
            setattr(self.cfg, k, v)
        c, rng = self.cfg, np.random.default_rng(seed)
        nq, nkv = c.heads * c.head_dim, c.kv_heads * c.head_dim
        w = lambda o, i: nlgpu.pack_ternary(rng.integers(-1, 2, (o, i))).ravel()
        sc = lambda i, n: np.full(n, 1 / np.sqrt(i / 2), f32)
        self.T = {}
        for l in range(c.layers):
            self.T.update({("wqkv", l): w(nq + 2 * nkv, c.d_model), ("bqkv", l): sc(c.d_model, nq + 2 * nkv),
                           ("wo", l): w(c.d_model, nq), ("bo", l): sc(nq, 1),
                           ("wgu", l): w(2 * c.d_ff, c.d_model), ("bgu", l): sc(c.d_model, 2 * c.d_ff),
                           ("wd", l): w(c.d_model, c.d_ff), ("bd", l): sc(c.d_ff, 1),
                           ("gattn", l): np.ones(c.d_model, f32), ("gffn", l): np.ones(c.d_model, f32)})
        half = c.head_dim // 2
        p = np.arange(c.max_seq)[:, None] / (500000.0 ** (2.0 * np.arange(half)[None, :] / c.head_dim))
        self.T.update({("wlm", -1): w(c.vocab, c.d_model), ("blm", -1): sc(c.d_model, 1),
                       ("gfinal", -1): np.ones(c.d_model, f32),
                       ("emb", -1): rng.standard_normal(c.vocab * c.d_model).astype(f32),
                       ("rope_cos", -1): np.cos(p).astype(f32).ravel(),
                       ("rope_sin", -1): np.sin(p).astype(f32).ravel()})

    def tensor(self, name, layer=-1, dtype=np.float32):
        return self.T[(name, layer)].view(dtype)


def test_one_lane_flip_moves_logits_by_percent(monkeypatch):
    """The decoder composition changed only in its RMSNorm sum order: the
    logits agree to ~1e-7 until an int8 lane crosses a rounding boundary,
    then differ by up to a few 1e-2 of max|logit| (carried on by the KV
    cache).  This is the scale the device stack's tolerance is set from."""
    cfg = dict(layers=2, d_model=256, heads=4, kv_heads=2, head_dim=64, d_ff=512, vocab=1000,
               max_seq=40, batch=2, rms_eps=1e-5)
    hs = _HostStack(**cfg)

    def rms64(x, gain, eps, rows, cols):
        x = np.asarray(x, f32).reshape(rows, cols)
        ss = (x.astype(np.float64) ** 2).sum(axis=1).astype(f32)
        s = (f32(1) / np.sqrt(ss / f32(cols) + f32(eps))).astype(f32)
        return ((x * s[:, None]).astype(f32) * gain).astype(f32).ravel()

    serial, reordered = ref.RefStack(hs), ref.RefStack(hs)
    tok, errs = np.array([3, 7]), []
    for pos in range(30):
        a = serial.step(tok, pos)
        monkeypatch.setattr(ref, "rms", rms64)
        b = reordered.step(tok, pos)
        monkeypatch.undo()
        errs.append(np.abs(a - b).max() / np.abs(a).max())
        tok = np.argmax(a, axis=1)
    errs = np.array(errs)
    print("max per step:", np.array2string(errs, precision=1))
    assert errs.max() < 5e-2
    first = int(np.argmax(errs > 1e-5)) if (errs > 1e-5).any() else len(errs)
    assert np.all(errs[:first] < 1e-6)  # before the first flip: rounding-level agreement


def test_paged_f16_attention_against_float64():
    """or_decode_attn_paged_f16 (decode-attn-paged-v over fp16 pools) against
    a float64 gather through the block table: shared blocks, a block
    outside the pool (zero rows), a non-power-of-two block size."""
    rng = np.random.default_rng(7)
    B, heads, kvh, hd, bs, mbps, npool = 3, 4, 2, 64, 7, 5, 12
    kvdim = kvh * hd
    kp = rng.standard_normal(npool * bs * kvdim).astype(np.float16)
    vp = rng.standard_normal(npool * bs * kvdim).astype(np.float16)
    table = rng.integers(0, npool, (B, mbps)).astype(np.int32)
    table[1, :2] = table[0, :2]  # a shared prefix
    table[2, 3] = npool + 5      # outside the pool
    lens = np.array([4, 30, 34], np.int32)
    q = rng.standard_normal(B * heads * hd).astype(np.float32)
    got = orc.decode_attn_paged_f16(q, kp.view(np.uint16), vp.view(np.uint16), lens, table, npool, B, heads, kvh,
                                    hd, bs, mbps).reshape(B, heads, hd)
    K = kp.astype(np.float64).reshape(npool, bs, kvh, hd)
    V = vp.astype(np.float64).reshape(npool, bs, kvh, hd)
    for s in range(B):
        n = lens[s] + 1
        for h in range(heads):
            kk, vv = np.zeros((n, hd)), np.zeros((n, hd))
            for j in range(n):
                ph = table[s, j // bs]
                if 0 <= ph < npool:
                    kk[j], vv[j] = K[ph, j % bs, h // (heads // kvh)], V[ph, j % bs, h // (heads // kvh)]
            sc = kk @ q.reshape(B, heads, hd)[s, h].astype(np.float64) / np.sqrt(hd)
            e = np.exp(sc - sc.max())
            want = (e[:, None] * vv).sum(axis=0) / e.sum()
            assert np.abs(got[s, h] - want).max() <= 1e-5 * max(1.0, np.abs(want).max())


def _ring_history(rng, B, kvh, hd, nsink, win, pos):
    """Stream positions 0..pos[s] appended one by one into fp16 ring caches
    with the reference's slot rule (later positions overwrite ring slots);
    returns the caches and, per sequence, every appended raw K/V row."""
    cap = nsink + win
    kc = np.zeros(B * kvh * cap * hd, np.uint16)
    vc = np.zeros_like(kc)
    hist = []
    for s in range(B):
        ks = rng.standard_normal((int(pos[s]) + 1, kvh * hd)).astype(f32)
        vs = rng.standard_normal((int(pos[s]) + 1, kvh * hd)).astype(f32)
        for p in range(int(pos[s]) + 1):
            pp = np.full(B, -1, np.int32)
            pp[s] = p
            orc.cache_append_ring_f16(kc, np.tile(ks[p], B), pp, B, kvh, hd, nsink, win)
            orc.cache_append_ring_f16(vc, np.tile(vs[p], B), pp, B, kvh, hd, nsink, win)
        hist.append((ks, vs))
    return kc, vc, hist


def test_ring_f16_attention_against_float64():
    """or_decode_attn_stream_f16 (decode-attn-stream over fp16 ring caches)
    against float64 attention over the positions a StreamingLLM cache keeps
    (the nsink first ones and the last win), built from the append history
    rather than from the ring-offset arithmetic; K rotated by its rank in that
    list and q by min(pos, cap - 1), pairs (2m, 2m+1)."""
    rng = np.random.default_rng(11)
    for B, heads, kvh, hd, nsink, win, pos in ((3, 4, 2, 64, 2, 6, [3, 7, 20]), (2, 2, 1, 128, 0, 5, [12, 4]),
                                               (2, 4, 1, 64, 4, 1, [2, 9])):
        pos = np.array(pos, np.int32)
        cap = nsink + win
        kc, vc, hist = _ring_history(rng, B, kvh, hd, nsink, win, pos)
        ang = np.outer(np.arange(cap), 1.0 / 10000.0 ** (np.arange(hd // 2) * 2.0 / hd))
        co, si = np.cos(ang).astype(f32), np.sin(ang).astype(f32)
        q = rng.standard_normal(B * heads * hd).astype(f32)
        got = orc.decode_attn_stream_f16(q, kc, vc, pos, co, si, B, heads, kvh, hd, nsink,
                                         win).reshape(B, heads, hd)
        for s in range(B):
            p = int(pos[s])
            kept = list(range(p + 1)) if p < cap else list(range(nsink)) + list(range(p - win + 1, p + 1))
            ks, vs = hist[s]
            qr = min(p, cap - 1)
            for h in range(heads):
                kv = h // (heads // kvh)
                qh = q.reshape(B, heads, hd)[s, h].astype(np.float64)
                q0, q1 = qh[0::2], qh[1::2]
                c, sn = co.astype(np.float64), si.astype(np.float64)
                qrot0, qrot1 = q0 * c[qr] - q1 * sn[qr], q0 * sn[qr] + q1 * c[qr]
                sc, vv = [], []
                for r, ap in enumerate(kept):
                    kk = ks[ap, kv * hd:(kv + 1) * hd].astype(np.float16).astype(np.float64)
                    k0, k1 = kk[0::2], kk[1::2]
                    kr0, kr1 = k0 * c[r] - k1 * sn[r], k0 * sn[r] + k1 * c[r]
                    sc.append((qrot0 @ kr0 + qrot1 @ kr1) / np.sqrt(hd))
                    vv.append(vs[ap, kv * hd:(kv + 1) * hd].astype(np.float16).astype(np.float64))
                e = np.exp(np.array(sc) - max(sc))
                want = (e @ np.array(vv)) / e.sum()
                assert np.abs(got[s, h] - want).max() <= 1e-5 * max(1.0, np.abs(want).max()), (B, s, h, p)


def test_ring_f16_attention_equals_the_dsl_restatement_bit_for_bit():
    """At one sequence the fp16 ring restatement performs the DSL kernel's
    operations in its order on the same (fp16-exact) values, so it matches
    decode-attn-stream's restatement on the reference's f32 [cap][kvdim]
    layout bit for bit, wrapped or not."""
    rng = np.random.default_rng(12)
    heads, kvh, hd, nsink, win = 4, 2, 64, 3, 5
    cap, kvd = nsink + win, kvh * hd
    co = rng.uniform(-1, 1, (cap, hd // 2)).astype(f32)
    si = rng.uniform(-1, 1, (cap, hd // 2)).astype(f32)
    for p in (0, 2, 6, 7, 8, 19):
        kc16 = rng.standard_normal(kvh * cap * hd).astype(np.float16)
        vc16 = rng.standard_normal(kvh * cap * hd).astype(np.float16)
        q = rng.standard_normal(heads * hd).astype(f32)
        got = orc.decode_attn_stream_f16(q, kc16.view(np.uint16), vc16.view(np.uint16), np.array([p], np.int32),
                                         co, si, 1, heads, kvh, hd, nsink, win)
        # the reference layout: slot-major rows of kvdim
        kref = kc16.astype(f32).reshape(kvh, cap, hd).transpose(1, 0, 2).reshape(cap * kvd).copy()
        vref = vc16.astype(f32).reshape(kvh, cap, hd).transpose(1, 0, 2).reshape(cap * kvd).copy()
        out = np.zeros(heads * hd, f32)
        orc.dispatch("decode-attn-stream", [q, kref, vref, np.array([p], f32), co.ravel(), si.ravel(), out],
                     [heads * hd, heads, kvh, nsink, win], (heads * hd + 63) // 64)
        assert np.array_equal(got.view(np.uint32), out.view(np.uint32)), p


def test_ring_f16_identity_rotation_is_plain_decode_attention():
    """With cos 1 and sin 0 and the ring not yet wrapped, ranks are positions
    and slots: the ring attention is decode-attn over the same cache."""
    rng = np.random.default_rng(13)
    B, heads, kvh, hd, nsink, win, pos = 2, 4, 1, 64, 2, 14, 9
    cap = nsink + win
    kc = rng.standard_normal(B * kvh * cap * hd).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal(B * kvh * cap * hd).astype(np.float16).view(np.uint16)
    q = rng.standard_normal(B * heads * hd).astype(f32)
    one, zero = np.ones((cap, hd // 2), f32), np.zeros((cap, hd // 2), f32)
    got = orc.decode_attn_stream_f16(q, kc, vc, np.full(B, pos, np.int32), one, zero, B, heads, kvh, hd, nsink, win)
    want = orc.decode_attn_f16(q, kc, vc, pos, B, heads, kvh, hd, cap)
    assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max()


def test_entries_f16_attention_equals_the_dsl_restatement_bit_for_bit():
    """or_attn_entries_f16 at one sequence performs attn-stream-entries'
    operations in its order on the same (fp16-exact) values: bit for bit the
    DSL restatement over the reference's f32 [nslots][kvdim] layout (entry
    base = slot * kvdim)."""
    rng = np.random.default_rng(14)
    heads, kvh, hd, nslots, trows = 4, 2, 64, 12, 20
    kvd = kvh * hd
    co = rng.uniform(-1, 1, (trows, hd // 2)).astype(f32)
    si = rng.uniform(-1, 1, (trows, hd // 2)).astype(f32)
    for ne, qr in ((1, 0), (7, 9), (12, 19)):
        kc16 = rng.standard_normal(kvh * nslots * hd).astype(np.float16)
        vc16 = rng.standard_normal(kvh * nslots * hd).astype(np.float16)
        ent = np.stack([rng.permutation(nslots)[:ne], rng.integers(0, trows, ne)], axis=1).astype(np.int32)
        q = rng.standard_normal(heads * hd).astype(f32)
        got = orc.attn_entries_f16(q, kc16.view(np.uint16), vc16.view(np.uint16), ent, np.array([qr], np.int32), co,
                                   si, 1, heads, kvh, hd, nslots, ne, trows)
        kref = kc16.astype(f32).reshape(kvh, nslots, hd).transpose(1, 0, 2).reshape(nslots * kvd).copy()
        vref = vc16.astype(f32).reshape(kvh, nslots, hd).transpose(1, 0, 2).reshape(nslots * kvd).copy()
        eref = np.stack([ent[:, 0] * kvd, ent[:, 1]], axis=1).astype(f32).ravel()
        out = np.zeros(heads * hd, f32)
        orc.dispatch("attn-stream-entries", [q, kref, vref, eref, co.ravel(), si.ravel(), out],
                     [heads * hd, heads, kvh, ne, qr], (heads * hd + 63) // 64)
        assert np.array_equal(got.view(np.uint32), out.view(np.uint32)), ne


def test_entries_f16_from_the_ring_rule_is_the_ring_attention():
    """An entry list spelling out the ring's (slot, rank) walk gives the ring
    attention's bits; a slot outside the cache counts as a zero row (score 0,
    V 0), checked against float64."""
    rng = np.random.default_rng(15)
    B, heads, kvh, hd, nsink, win = 2, 4, 2, 64, 3, 6
    cap = nsink + win
    kc = rng.standard_normal(B * kvh * cap * hd).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal(B * kvh * cap * hd).astype(np.float16).view(np.uint16)
    co = rng.uniform(-1, 1, (cap, hd // 2)).astype(f32)
    si = rng.uniform(-1, 1, (cap, hd // 2)).astype(f32)
    q = rng.standard_normal(B * heads * hd).astype(f32)
    pos = np.array([30, 30], np.int32)  # same stream position: entry lists of one length
    start = pos[0] - win + 1
    woff = (start - nsink) % win
    slots = [r if r < nsink else nsink + (woff + r - nsink) % win for r in range(cap)]
    ent = np.tile(np.stack([slots, np.arange(cap)], axis=1), (B, 1)).astype(np.int32)
    qrank = np.full(B, cap - 1, np.int32)
    got = orc.attn_entries_f16(q, kc, vc, ent, qrank, co, si, B, heads, kvh, hd, cap, cap, cap)
    want = orc.decode_attn_stream_f16(q, kc, vc, pos, co, si, B, heads, kvh, hd, nsink, win)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # an out-of-range slot: a zero K row (score 0) and a zero V row
    ent2 = ent.copy().reshape(B, cap, 2)
    ent2[0, 4, 0] = 1000
    got2 = orc.attn_entries_f16(q, kc, vc, ent2, qrank, co, si, B, heads, kvh, hd, cap, cap, cap).reshape(B, heads,
                                                                                                        hd)
    K = kc.view(np.float16).astype(np.float64).reshape(B, kvh, cap, hd)
    V = vc.view(np.float16).astype(np.float64).reshape(B, kvh, cap, hd)
    c, sn = co.astype(np.float64), si.astype(np.float64)
    for h in range(heads):
        kv = h // (heads // kvh)
        qh = q.reshape(B, heads, hd)[0, h].astype(np.float64)
        qr0 = qh[0::2] * c[cap - 1] - qh[1::2] * sn[cap - 1]
        qr1 = qh[0::2] * sn[cap - 1] + qh[1::2] * c[cap - 1]
        sc, vv = [], []
        for r in range(cap):
            sl, rk = ent2[0, r]
            if sl >= cap:
                sc.append(0.0)
                vv.append(np.zeros(hd))
                continue
            k = K[0, kv, sl]
            kr0, kr1 = k[0::2] * c[rk] - k[1::2] * sn[rk], k[0::2] * sn[rk] + k[1::2] * c[rk]
            sc.append((qr0 @ kr0 + qr1 @ kr1) / np.sqrt(hd))
            vv.append(V[0, kv, sl])
        e = np.exp(np.array(sc) - max(sc))
        w = (e @ np.array(vv)) / e.sum()
        assert np.abs(got2[0, h] - w).max() <= 1e-5 * max(1.0, np.abs(w).max())
