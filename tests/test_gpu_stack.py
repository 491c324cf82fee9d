"""The ternary decoder stack on the MI355X.

* Its device-drawn weights equal the host generator's (trits and gains
  exactly; the embedding's Box-Muller within 2 ulp, since the device's
  double log/sin/cos are not bit-pinned to libm's).
* Captured-graph steps give the same bits as eager steps.
* Prompt tokens are teacher-forced, then each token is the greedy choice of
  the step before it.
* Its logits follow the reference kernels chained on the CPU
  (tests/layer_ref.py) step by step.  The model's composition is this
  build's own (the reference's model code is not in its tree), so this is a
  tolerance check: the RMSNorm, attention and SiLU use device reductions and
  exp, whose last-bit differences can move an int8 activation lane across a
  rounding boundary now and then, and the KV cache carries that forward.
  Until the first such event the logits agree to ~1e-7 of max|logit|; after
  it they differ by 1e-2..3e-2 -- the same jump the CPU composition makes
  when only its RMSNorm sum order changes (test_oracle_layer.py
  test_one_lane_flip_moves_logits_by_percent).  The bar is 1e-5 for the first
  prompt steps and 5e-2 after.
* At batch 8 with head_dim 128 and three attention chunks (the batched
  decode path and the three-chunk merge), and at config 5's full size
  (30 layers, d_model 2560, vocab 128,256, a 512-token prompt, B = 1 and
  32): prefill against teacher-forced steps, graph replay against eager
  steps bit for bit, greedy consistency, and the next step checked a layer
  at a time against the CPU composition (each layer fed the device's own
  residual stream, so a lane flip shows in one layer only).
"""
import numpy as np
import pytest

import layer_ref as ref
import nlgpu

pytestmark = pytest.mark.gpu

TINY = dict(layers=2, d_model=256, heads=4, kv_heads=2, head_dim=64, d_ff=512, vocab=1000,
            max_seq=80, batch=2)


@pytest.fixture(scope="module", autouse=True)
def device():
    nlgpu.init()
    yield


def prompts(B, n, vocab, seed=5):
    return (nlgpu.uniform(seed, B * n) * vocab).astype(np.int32).reshape(B, n)


def test_weights_follow_the_host_generator():
    print("[gpu] stack generator", flush=True)
    s = nlgpu.Stack(**TINY, seed=123)
    c = s.cfg
    seed = lambda l, t: nlgpu.stack_tensor_seed(123, l, t)
    d, f, nq, nkv = c.d_model, c.d_ff, c.heads * c.head_dim, c.kv_heads * c.head_dim
    want = np.concatenate([nlgpu.pack_ternary(nlgpu.trits(seed(1, 0), (nq, d))),
                           nlgpu.pack_ternary(nlgpu.trits(seed(1, 1), (nkv, d))),
                           nlgpu.pack_ternary(nlgpu.trits(seed(1, 2), (nkv, d)))]).ravel()
    assert np.array_equal(s.tensor("wqkv", 1, np.uint32), want)
    gu = np.empty((2 * f, d // 16), np.uint32)
    gu[0::2] = nlgpu.pack_ternary(nlgpu.trits(seed(0, 4), (f, d)))
    gu[1::2] = nlgpu.pack_ternary(nlgpu.trits(seed(0, 5), (f, d)))
    assert np.array_equal(s.tensor("wgu", 0, np.uint32), gu.ravel())
    g = (0.75 + 0.5 * nlgpu.uniform(seed(0, 8), d)).astype(np.float32)
    assert np.array_equal(s.tensor("gffn", 0), g)
    emb = s.tensor("emb")
    want = nlgpu.normal_pairs(seed(c.layers, 2), c.vocab * d)
    assert np.all(np.abs(emb - want) <= 2 * np.spacing(np.abs(want)))
    s.close()


def test_graph_replay_matches_eager_and_greedy_is_consistent():
    print("[gpu] stack graph vs eager", flush=True)
    P = prompts(TINY["batch"], 4, TINY["vocab"])
    out = []
    for graph in (False, True):
        s = nlgpu.Stack(**TINY)
        s.start(P)
        s.step(10, graph=graph)
        toks, greedy = s.tokens()
        out.append((toks, greedy, s.logits()))
        s.close()
    (t0, g0, l0), (t1, g1, l1) = out
    assert np.array_equal(t0, t1) and np.array_equal(g0, g1)
    assert np.array_equal(l0.view(np.uint32), l1.view(np.uint32))
    assert np.array_equal(t0[:, :4], P)                 # prompt teacher-forced
    assert np.array_equal(t0[:, 4:11], g0[:, 3:10])     # then greedy
    assert np.array_equal(g0[:, 9], np.argmax(l0, axis=1))
    assert np.all(t0[:, 11:] == -1)


def test_logits_follow_the_reference_kernels():
    print("[gpu] stack vs chained reference kernels", flush=True)
    s = nlgpu.Stack(**TINY)
    r = ref.RefStack(s)
    P = prompts(TINY["batch"], 3, TINY["vocab"], seed=9)
    s.start(P)
    worst = 0.0
    for pos in range(12):
        toks, _ = s.tokens()
        want = r.step(toks[:, pos], pos)
        s.step(1)
        got = s.logits()
        err = np.abs(got - want).max() / np.abs(want).max()
        worst = max(worst, err)
        print(f"  pos={pos} max|dlogit|/max|logit| = {err:.2e}", flush=True)
        assert err <= (1e-5 if pos < 2 else 5e-2)
    print(f"  worst {worst:.2e}")
    s.close()


@pytest.mark.parametrize("n", [12, 64])
def test_prefill_matches_teacher_forced_steps(n):
    """All prompt rows at once (batched linears -- the 128 x 128 matrix-core
    tiles from 128 rows on -- and causal attention over the cache) against
    the same prompt fed one token per step: same state, and logits / caches
    within the lane-flip bar (the two paths round RMSNorm's sum in different
    orders)."""
    print(f"[gpu] stack prefill vs teacher-forced steps, prompt {n}", flush=True)
    P = prompts(TINY["batch"], n, TINY["vocab"], seed=11)
    a, b = nlgpu.Stack(**TINY), nlgpu.Stack(**TINY)
    a.start(P)
    a.step(n, graph=False)
    b.prefill(P)
    assert a.position() == b.position() == n
    la, lb = a.logits(), b.logits()
    err = np.abs(la - lb).max() / np.abs(la).max()
    print(f"  logits max|d|/max = {err:.2e}", flush=True)
    assert err <= 5e-2
    ta, ga = a.tokens()
    tb, gb = b.tokens()
    assert np.array_equal(tb[:, :n], P) and np.array_equal(ta[:, :n], P)
    assert np.array_equal(gb[:, n - 1], np.argmax(lb, axis=1)) and np.array_equal(tb[:, n], gb[:, n - 1])
    assert np.all(gb[:, :n - 1] == -1)
    c = a.cfg
    for l in range(c.layers):
        for name in ("kc", "vc"):
            ka = a.tensor(name, l, np.float16).reshape(c.batch, c.kv_heads, c.max_seq, c.head_dim)[:, :, :n]
            kb = b.tensor(name, l, np.float16).reshape(c.batch, c.kv_heads, c.max_seq, c.head_dim)[:, :, :n]
            d = np.abs(ka.astype(np.float32) - kb.astype(np.float32)).max()
            assert d <= 5e-2 * np.abs(ka.astype(np.float32)).max(), (l, name, d)
    b.step(5)  # decoding continues from the prefilled state
    tb2, _ = b.tokens()
    assert np.array_equal(tb2[:, :n + 1], tb[:, :n + 1]) and np.all(tb2[:, n + 1:n + 6] >= 0)
    a.close()
    b.close()


# Batch >= 4 takes the batched decode path (per-token quantisation + the
# small-batch GEMM epilogues, batched argmax partials); head_dim 128 with
# max_seq in (512, 768] gives three attention chunks, merged by the
# three-chunk prologue of the output projection.
MID = dict(layers=2, d_model=512, heads=4, kv_heads=2, head_dim=128, d_ff=1024, vocab=1000, max_seq=700,
           batch=8)


@pytest.mark.parametrize("B", [8, 5])
def test_batched_decode_graph_eager_and_reference(B):
    print(f"[gpu] stack B={B} hd=128 max_seq=700: graph vs eager, greedy, reference", flush=True)
    vocab = MID["vocab"]
    kw = dict(MID, batch=B)
    P = prompts(B, 3, vocab, seed=31)
    a, b = nlgpu.Stack(**kw), nlgpu.Stack(**kw)
    r = ref.RefStack(a)
    a.start(P)
    b.start(P)
    for pos in range(10):
        toks, _ = a.tokens()
        want = r.step(toks[:, pos], pos)
        a.step(1, graph=False)
        err = np.abs(a.logits() - want).max(axis=1) / np.abs(want).max(axis=1)
        print(f"  pos={pos} max|dlogit|/max|logit| per sequence = {np.array2string(err, precision=1)}", flush=True)
        # A lane that crosses a rounding boundary (the device's tree sums vs
        # the reference's serial ones) moves one sequence's logits by ~1e-2
        # and the cache carries it on; a systematic error would move them all.
        assert np.all(err <= 5e-2)
        if pos < 3:
            assert np.sum(err <= 1e-5) >= B // 2, err
    b.step(10, graph=True)
    (ta, ga), (tb, gb) = a.tokens(), b.tokens()
    assert np.array_equal(ta, tb) and np.array_equal(ga, gb)
    assert np.array_equal(a.logits().view(np.uint32), b.logits().view(np.uint32))
    assert np.array_equal(ta[:, :3], P) and np.array_equal(ta[:, 3:11], ga[:, 2:10])
    a.close()
    b.close()


def _write_weights(s, name, layer, words):
    """Write 2-bit weight words into a stack tensor through the device
    pointer nlg_stack_tensor hands out."""
    import ctypes as C
    p, n = C.c_void_p(), C.c_size_t(0)
    L = nlgpu.lib()
    assert L.nlg_stack_tensor(s.h, name.encode(), layer, C.byref(p), C.byref(n)) == 0
    w = np.ascontiguousarray(words, np.uint32)
    assert w.nbytes == n.value
    assert L.nlg_upload(p.value, w.ctypes.data, w.nbytes) == 0


def test_weights_written_through_tensor_pointers():
    """Weights written through the pointers nlg_stack_tensor hands out reach
    the matrix-core linears, which read tiled copies (batch 8: the decode
    step's linears; prefill): the stack refreshes the copies before its next
    prefill or step.  Checked against the CPU composition reading the new
    weights (a stale copy would put the logits O(1) off), graph replay
    against eager bits, and prefill against teacher-forced steps."""
    print("[gpu] stack B=8: weights written through tensor pointers", flush=True)
    B, n = MID["batch"], 3
    c = MID
    d, f, nq, nkv = c["d_model"], c["d_ff"], c["heads"] * c["head_dim"], c["kv_heads"] * c["head_dim"]
    new = {("wqkv", 0): nlgpu.pack_ternary(nlgpu.trits(901, (nq + 2 * nkv, d))),
           ("wd", 1): nlgpu.pack_ternary(nlgpu.trits(902, (d, f))),
           ("wlm", -1): nlgpu.pack_ternary(nlgpu.trits(903, (c["vocab"], d)))}
    P = prompts(B, n, c["vocab"], seed=35)
    a, b, e = nlgpu.Stack(**MID), nlgpu.Stack(**MID), nlgpu.Stack(**MID)
    for st in (a, b, e):
        for (name, layer), w in new.items():
            _write_weights(st, name, layer, w)
    for (name, layer), w in new.items():
        assert np.array_equal(a.tensor(name, layer, np.uint32), w.ravel())
    r = ref.RefStack(a)
    a.start(P)
    b.start(P)
    for pos in range(6):
        toks, _ = a.tokens()
        want = r.step(toks[:, pos], pos)
        a.step(1, graph=False)
        err = np.abs(a.logits() - want).max(axis=1) / np.abs(want).max(axis=1)
        print(f"  pos={pos} max|dlogit|/max|logit| per sequence = {np.array2string(err, precision=1)}", flush=True)
        assert np.all(err <= 5e-2)
        if pos < 3:
            assert np.sum(err <= 1e-5) >= B // 2, err
    b.step(6, graph=True)
    assert np.array_equal(a.logits().view(np.uint32), b.logits().view(np.uint32))
    e.prefill(P)
    t = nlgpu.Stack(**MID)
    for (name, layer), w in new.items():
        _write_weights(t, name, layer, w)
    t.start(P)
    t.step(n, graph=False)
    lt, le = t.logits(), e.logits()
    err = np.abs(lt - le).max() / np.abs(lt).max()
    print(f"  prefill vs teacher-forced logits max|d|/max = {err:.2e}", flush=True)
    assert err <= 5e-2
    for st in (a, b, e, t):
        st.close()


def test_batched_decode_after_long_prefill():
    """A 600-token prompt (three chunks in use) prefilled at once against the
    same prompt teacher-forced, then decode steps: graph == eager bits,
    greedy consistency, and the next step's logits against the reference
    composition started from the device's caches."""
    print("[gpu] stack B=8 prefill 600 vs teacher-forced, then decode", flush=True)
    n, B = 600, MID["batch"]
    P = prompts(B, n, MID["vocab"], seed=33)
    a, b, c = nlgpu.Stack(**MID), nlgpu.Stack(**MID), nlgpu.Stack(**MID)
    a.prefill(P)
    c.prefill(P)
    b.start(P)
    b.step(n, graph=True)
    assert a.position() == b.position() == n
    la, lb = a.logits(), b.logits()
    err = np.abs(la - lb).max() / np.abs(lb).max()
    print(f"  prefill vs teacher-forced logits max|d|/max = {err:.2e}", flush=True)
    assert err <= 5e-2
    r = ref.RefStack(a)
    r.load_caches(a, n)
    ta, _ = a.tokens()
    want = r.step(ta[:, n], n)
    a.step(1, graph=False)
    err = np.abs(a.logits() - want).max() / np.abs(want).max()
    print(f"  step at {n} vs reference from the same caches: {err:.2e}", flush=True)
    assert err <= 5e-2
    a.step(4, graph=False)
    c.step(5, graph=True)
    (ta, ga), (tc, gc) = a.tokens(), c.tokens()
    assert np.array_equal(ta, tc) and np.array_equal(ga, gc)
    assert np.array_equal(a.logits().view(np.uint32), c.logits().view(np.uint32))
    assert np.array_equal(ta[:, n + 1:n + 6], ga[:, n:n + 5])
    for s in (a, b, c):
        s.close()


# Config 5 at its real size: 30 layers, d_model 2560, 20/5 heads of 128,
# d_ff 6912, vocab 128,256, 512-token prompts, B = 1 and 32.
FULL = dict(layers=30, d_model=2560, heads=20, kv_heads=5, head_dim=128, d_ff=6912, vocab=128256, max_seq=768)


@pytest.mark.parametrize("B", [1, 32])
def test_config5_full_size(B):
    n = 512
    print(f"[gpu] config 5 full size B={B}: prefill {n}, teacher-forced, decode", flush=True)
    P = prompts(B, n, FULL["vocab"], seed=41)
    a, c = nlgpu.Stack(**FULL, batch=B), nlgpu.Stack(**FULL, batch=B)
    a.prefill(P)
    c.prefill(P)
    # the same prompt one token per step (teacher-forced) in a third stack
    b = nlgpu.Stack(**FULL, batch=B)
    b.start(P)
    b.step(n, graph=True)
    assert a.position() == b.position() == n
    # The two paths round RMSNorm's sums of squares in different orders, so
    # now and then an int8 lane lands on the other side of a rounding
    # boundary (~1e-2 of one output), and at 30 layers x 512 positions those
    # flips cascade through attention and the residual stream: layer 0's
    # caches agree to a few fp16 ulps, deeper layers drift to ~6e-2 of their
    # range and the logits to ~6e-2 of max|logit| (cosine ~0.998) -- the
    # accumulated lane-flip floor of an int8-quantised network, not a
    # systematic error (the single-step check against the CPU reference
    # below, from identical caches, agrees to ~1e-7 until a flip).
    la, lb = a.logits(), b.logits()
    err = np.abs(la - lb).max() / np.abs(lb).max()
    cos = np.min(np.sum(la * lb, axis=1) / np.linalg.norm(la, axis=1) / np.linalg.norm(lb, axis=1))
    print(f"  prefill vs teacher-forced logits max|d|/max = {err:.2e}, min cosine {cos:.6f}", flush=True)
    assert err <= 1.5e-1 and cos >= 0.99
    cfg = a.cfg
    for l, bar in ((0, 2e-3), (cfg.layers - 1, 1.5e-1)):
        for name in ("kc", "vc"):
            ka = a.tensor(name, l, np.float16).reshape(B, cfg.kv_heads, cfg.max_seq, cfg.head_dim)[:, :, :n]
            kb = b.tensor(name, l, np.float16).reshape(B, cfg.kv_heads, cfg.max_seq, cfg.head_dim)[:, :, :n]
            d = np.abs(ka.astype(np.float32) - kb.astype(np.float32)).max()
            print(f"  layer {l} {name}: max|d|/max = {d / np.abs(kb.astype(np.float32)).max():.2e}", flush=True)
            assert d <= bar * np.abs(kb.astype(np.float32)).max(), (l, name, d)
    b.close()
    # The next step, one layer at a time, against the reference kernels
    # chained on the CPU (two sequences of the batch: they are independent):
    # the reference starts from the device's caches, and each layer takes the
    # device's residual stream as its input, so a lane flip stays in the
    # layer it happens in instead of cascading through the rest.
    seqs = [0, B - 1] if B > 1 else [0]
    r = ref.RefStack(a, seqs=seqs)
    r.load_caches(a, n)
    ta, _ = a.tokens()
    xs = a.step_trace()[:, seqs]
    assert np.array_equal(xs[0].view(np.uint32), r.embed(ta[seqs, n]).view(np.uint32))
    errs = []
    for l in range(cfg.layers):
        want = r.layer(l, xs[l], n)
        errs.append(np.abs(xs[l + 1] - want).max() / np.abs(want).max())
    want = r.head(xs[cfg.layers])
    errs.append(np.abs(a.logits()[seqs] - want).max() / np.abs(want).max())
    del r
    errs = np.array(errs)
    print(f"  step at {n}, per layer (then the head) vs reference: median {np.median(errs):.2e}, "
          f"max {errs.max():.2e}, {np.sum(errs > 1e-5)} of {errs.size} above 1e-5", flush=True)
    # a flip moves one layer by ~1e-2; a systematic error would move them all
    assert errs.max() <= 5e-2 and np.median(errs) <= 1e-5
    # graph replay == eager, bit for bit; greedy consistency
    a.step(3, graph=False)
    c.step(4, graph=True)
    (ta, ga), (tc, gc) = a.tokens(), c.tokens()
    assert np.array_equal(ta, tc) and np.array_equal(ga, gc)
    assert np.array_equal(a.logits().view(np.uint32), c.logits().view(np.uint32))
    assert np.array_equal(ta[:, :n], P) and np.array_equal(ta[:, n + 1:n + 5], ga[:, n:n + 4])
    assert np.all(ta[:, n + 5:] == -1)
    a.close()
    c.close()


def test_config5_prefill_layers_against_reference():
    """Config 5's prefill (B = 1, a 512-token prompt: batched int8 linears,
    split prompt attention merged and quantised for the output projection)
    checked a layer at a time against the reference kernels chained on the
    CPU: for layers 0, 15 and 29 and prompt rows 0, 1, 255 and 511, the
    reference's decode step at that row's position, fed the device's input
    rows of that layer and the device's caches of the positions before the
    row, against the device's output rows.  A lane flip moves one check by
    ~1e-2; a systematic error would move them all (bar: median <= 1e-5,
    max <= 5e-2, as for the decode step)."""
    n, B = 512, 1
    print(f"[gpu] config 5 full size B={B}: prefill {n} layer by layer vs reference", flush=True)
    P = prompts(B, n, FULL["vocab"], seed=43)
    a = nlgpu.Stack(**FULL, batch=B)
    xs = a.prefill_trace(P)
    cfg = a.cfg
    assert xs.shape == (cfg.layers + 1, n, cfg.d_model)
    r = ref.RefStack(a)
    assert np.array_equal(xs[0].view(np.uint32), r.emb[P[0]].astype(np.float32).view(np.uint32))
    errs = []
    for l in (0, 15, cfg.layers - 1):
        for row in (0, 1, 255, n - 1):
            r.load_caches(a, row, layers=[l])
            want = r.layer(l, xs[l][row:row + 1], row)
            e = float(np.abs(xs[l + 1][row] - want[0]).max() / np.abs(want).max())
            print(f"  layer {l:2d} row {row:3d}: max|d|/max = {e:.2e}", flush=True)
            errs.append(e)
    del r
    errs = np.array(errs)
    assert errs.max() <= 5e-2 and np.median(errs) <= 1e-5, errs
    # the prefilled state decodes on
    a.step(2)
    t, g = a.tokens()
    assert np.array_equal(t[:, :n], P) and np.array_equal(t[:, n + 1:n + 3], g[:, n:n + 2])
    a.close()

