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
