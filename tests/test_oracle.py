"""Pin the CPU restatement (oracle/nlg_oracle.c) before trusting it.

Every kernel of the table is run through the oracle and checked against an
independent statement (tests/np_ref.py: float64 closed forms, vectorised
float32 restatements from the layouts, int64 brute force), and the hot-path
pieces get known-answer tests chosen so a plausible slip -- a wrong field
order, a missing sign extension, a dropped rounding half, a transposed
operand -- fails: the 2-bit decode words, the int8 rounding ties and clamp,
the reference test's own LCG vectors (test/ternary-kernel-test.el) with its
1e-5 bar and block-scale control, vkmatmul's integer known answer
(host/vkmatmul.c:92-93), and closed-form special cases of softmax, RoPE and
attention.  No GPU needed.
"""
import numpy as np
import pytest

import kernel_specs as ks
import nlg_oracle as orc
import nlgpu
import np_ref

# np_ref states these as exact float32/int sequences: bitwise pin
EXACT_PIN = {"vadd", "add2", "mul", "scale", "causal-mask", "rmsnorm-fwd", "embed-gather",
             "cache-append", "cache-append-b", "qkv-append", "decode-rope", "decode-rope-b",
             "rope-apply", "pack-act-rows", "quant-act", "dp4a-dot", "bitlinear-dp4a",
             "bitlinear-dp4a-1f", "bitlinear-dp4a-rows", "cache-append-ring", "cache-append-paged",
             "cache-append-paged-v", "block-copy", "decode-rope-b-v"}
PIN_TOL = {"softmax": ks.ELEM(1e-5), "silu": 1e-6, "silu-mul": 1e-6, "rmsnorm-istd": 1e-5,
           "rmsnorm-heads": 1e-5, "rope-half": 1e-5, "ternary-rows": 1e-5, "bitlinear-packed": 1e-5,
           "bitlinear-packed-v": 1e-5, "matmul": 1e-5, "matmul-tiled": 1e-5, "matmul-reg": 1e-5,
           "linear": 1e-5, "attn-scores": 1e-5, "attn-context": 1e-5, "decode-attn": 1e-5,
           "decode-attn-b": 1e-5, "attn-causal-gqa": 1e-5, "decode-attn-stream": 1e-5,
           "attn-stream-entries": 1e-5, "decode-attn-paged": 1e-5, "decode-attn-paged-v": 1e-5,
           "ternary-rows-t": 1e-5, "dp4a-rows-t": 1e-5}

CASES = ks.cases()


def run_oracle(case):
    bufs = []
    for i, b in enumerate(case.bufs):
        bufs.append(bufs[case.alias[i]] if i in case.alias else np.array(b, copy=True))
    orc.dispatch(case.name, bufs, case.push, case.groups)
    return bufs


@pytest.mark.parametrize("case", CASES, ids=[ks.case_id(c) for c in CASES])
def test_oracle_matches_independent_statement(case):
    got = run_oracle(case)
    want = np_ref.ref(case)
    tol = ks.EXACT if case.name in EXACT_PIN else PIN_TOL[case.name]
    for idx, w in want.items():
        ok, err = np_ref.compare(got[idx], w, tol)
        assert ok, f"{ks.case_id(case)} buffer {idx}: error {err} (bar {tol})"
    # inputs that are not outputs are untouched
    for i, b in enumerate(case.bufs):
        if i not in want and i not in case.alias and not any(case.alias.get(j) == i for j in want):
            assert np.array_equal(got[i].view(np.uint32), np.asarray(b).view(np.uint32)), (case.name, i)


def test_every_table_kernel_has_a_case():
    assert set(orc.kernel_names()) == {c.name for c in CASES}


# --------------------------------------------------------------- int8 quantisation

def _pack(x, cols=None):
    x = np.asarray(x, np.float32)
    cols = x.size if cols is None else cols
    return orc.pack_act_rows(x, 1, cols)


def test_pack_act_known_answers():
    # amax = 127 gives gamma = 1 exactly: lanes are round-half-up of |x|
    xq, g = _pack([127.0, -127.0, 2.5, -2.5, 0.49, -0.5, 1.5, 0.0])
    assert g[0] == np.float32(1.0)
    lanes = xq.view(np.uint8)
    assert list(lanes) == [127, 0x81, 3, 256 - 3, 0, 255, 2, 0]
    # all-zero row: gamma 0, every lane 0 (kernels.el:914 guards the division)
    xq, g = _pack(np.zeros(13, np.float32))
    assert g[0] == 0.0 and not xq.any() and xq.size == 4
    # +-amax map to +-127 for any scale
    xq, g = _pack([3.7e-3, -3.7e-3, 1e-3])
    assert list(xq.view(np.uint8)[:2]) == [127, 0x81]
    # the clamp: a subnormal amax makes gamma round to one subnormal step,
    # so |x|/gamma = 190 and only the min(ri, 127) keeps the lane in range
    step = np.float32(2.0 ** -149)
    xq, g = _pack([np.float32(190) * step])
    assert g[0] == step and xq.view(np.uint8)[0] == 127
    # a NaN never wins the max (ordered compare), and -0 packs as 0
    xq, g = _pack([np.nan, 2.0, -0.0, -1.0])
    assert g[0] == np.float32(2.0) / np.float32(127.0)
    assert list(xq.view(np.uint8)[1:]) == [127, 0, 256 - 64]


def test_quant_act_equals_gamma_times_packed_lanes():
    rng = np.random.default_rng(7)
    seq, cols = 4, 333
    x = (rng.standard_normal(seq * cols) * 3).astype(np.float32)
    xq, gamma = orc.pack_act_rows(x, seq, cols)
    lanes = xq.view(np.int8).reshape(seq, -1)[:, :cols].astype(np.float32)
    fq = np.zeros(seq * cols, np.float32)
    orc.dispatch("quant-act", [x.copy(), fq], [seq, cols], 1)
    # quant-act writes gamma*sgn*min(round,127): the same rounding as the packed lane
    want = (gamma[:, None] * lanes).astype(np.float32)
    # a negative x that rounds to lane 0 gives gamma*(-1*0) = -0.0 (sgn is -1)
    xs = x.reshape(seq, cols)
    want = np.where(lanes == 0, np.where(xs < 0, np.float32(-0.0), np.float32(0.0)), want)
    assert np.array_equal(fq.reshape(seq, cols).view(np.uint32), want.view(np.uint32))


# --------------------------------------------------------------- 2-bit decode

@pytest.mark.parametrize("word,field,value", [
    (0x00000001, 0, +1), (0x00000003, 0, -1), (0x00000002, 0, -2), (0x00000000, 0, 0),
    (0xC0000000, 15, -1), (0x40000000, 15, +1), (0x80000000, 15, -2), (0x0000000C, 1, -1),
    (0x00000004, 1, +1), (0x00300000, 10, -1)])
def test_two_bit_decode_known_words(word, field, value):
    # one output row, 16 columns; x = +1 at `field` only (lane value 1)
    cols = 16
    x = np.zeros(cols, np.int8)
    x[field] = 1
    xq = x.view(np.uint8).view(np.uint32)
    acc = orc.ternary_acc_i8(xq, np.array([word], np.uint32), 1, 1, cols)
    assert acc[0] == value
    # and every other field of the word is 0 or ignored by a zero activation
    assert nlgpu.unpack_ternary(np.array([[word]], np.uint32), 16)[0, field] == value


def test_pack_unpack_round_trip():
    rng = np.random.default_rng(3)
    t = rng.integers(-2, 2, (7, 53)).astype(np.int8)
    assert np.array_equal(nlgpu.unpack_ternary(nlgpu.pack_ternary(t), 53), t)


@pytest.mark.parametrize("seq,out,cols", [(1, 17, 16), (3, 9, 100), (2, 5, 4096), (1, 3, 1), (2, 4, 37)])
def test_ternary_acc_brute_force(seq, out, cols):
    rng = np.random.default_rng(seq * 1000 + cols)
    t = rng.integers(-2, 2, (out, cols)).astype(np.int8)  # includes the -2 code
    w2 = nlgpu.pack_ternary(t)
    x = (rng.standard_normal(seq * cols) * 2).astype(np.float32)
    xq, gamma = orc.pack_act_rows(x, seq, cols)
    xi = xq.view(np.int8).reshape(seq, -1)[:, :cols].astype(np.int64)
    want = (xi @ t.astype(np.int64).T).ravel()
    got = orc.ternary_acc_i8(xq, w2, seq, out, cols)
    assert np.array_equal(got, want)
    # garbage lanes past `cols` in the activation words must not leak in
    xq2 = xq.copy().view(np.uint8).reshape(seq, -1)
    xq2[:, cols:] = 0x7F
    assert np.array_equal(orc.ternary_acc_i8(xq2.view(np.uint32).ravel(), w2, seq, out, cols), want)


def test_ternary_linear_epilogue_and_dp4a_equivalence():
    rng = np.random.default_rng(11)
    seq, out, cols = 3, 21, 300
    t = rng.integers(-1, 2, (out, cols)).astype(np.int8)
    w2 = nlgpu.pack_ternary(t)
    x = rng.standard_normal(seq * cols).astype(np.float32)
    xq, gamma = orc.pack_act_rows(x, seq, cols)
    bias = rng.standard_normal(out).astype(np.float32)
    beta = np.array([0.0371], np.float32)
    y = orc.ternary_linear_i8(xq, gamma, w2, bias, beta, seq, out, cols)
    acc = orc.ternary_acc_i8(xq, w2, seq, out, cols).reshape(seq, out).astype(np.float32)
    want = bias[None, :] + (beta[0] * gamma[:, None]).astype(np.float32) * acc
    assert np.array_equal(y.view(np.uint32), want.astype(np.float32).ravel().view(np.uint32))
    # the composite is bitlinear-dp4a-1f on the weights unpacked to int8 lanes
    ng = (cols + 3) // 4
    w8 = np.zeros((out, ng * 4), np.int8)
    w8[:, :cols] = t
    yd = np.zeros(seq * out, np.float32)
    orc.dispatch("bitlinear-dp4a-1f", [xq.view(np.float32).copy(), w8.view(np.uint32).ravel().view(np.float32).copy(),
                                       bias.copy(), beta.copy(), gamma.copy(), yd], [seq, out, ng], 1)
    assert np.array_equal(yd.view(np.uint32), y.view(np.uint32))
    # per-row beta and a null bias
    betar = np.abs(rng.standard_normal(out)).astype(np.float32) * 0.05
    y2 = orc.ternary_linear_i8(xq, gamma, w2, None, betar, seq, out, cols, beta_per_row=True)
    want2 = np.float32(0) + (betar[None, :] * gamma[:, None]).astype(np.float32) * acc
    assert np.array_equal(y2.view(np.uint32), want2.astype(np.float32).ravel().view(np.uint32))


# --------------------------------------------------- the reference test's vectors

def _lcg_fixture():
    import os
    return np.load(os.path.join(os.path.dirname(__file__), "golden", "ternary_rows_lcg.npz"))


def _ternary_rows(d, beta):
    seq, out, cols, nblk, wng = (int(d[k]) for k in ("seq", "out", "cols", "nblk", "wng"))
    y = np.zeros(seq * out, np.float32)
    orc.dispatch("ternary-rows", [d["x"].astype(np.float32), d["wp"].view(np.float32).copy(),
                                  d["bias"].astype(np.float32), beta.astype(np.float32), y],
                 [seq, out, cols, nblk, wng], (seq * out + 63) // 64)
    return y


def test_ternary_rows_against_reference_test_vectors():
    d = _lcg_fixture()
    # the fixture's packing is the test's tk-pack; it must decode to its trits
    assert np.array_equal(nlgpu.unpack_ternary(d["wp"].reshape(6, 16), 256), d["trits"])
    y = _ternary_rows(d, d["beta"])
    want = d["y"]
    err = np.max(np.abs(y - want)) / np.max(np.abs(want))
    assert err < 1e-5, err  # tk-err bar (ternary-kernel-test.el:23-34, :109-110)
    assert np.any(y != 0)   # control: not all zero (:105-107)


def test_ternary_rows_block_scale_control():
    d = _lcg_fixture()
    y0 = _ternary_rows(d, d["beta"])
    b2 = d["beta"].copy()
    b2[1] *= 3.0  # row 0, second block only (ternary-kernel-test.el:160)
    y1 = _ternary_rows(d, b2).reshape(3, 6)
    y0 = y0.reshape(3, 6)
    assert np.all(y0[:, 0] != y1[:, 0])          # moves that row in every position
    assert np.array_equal(y0[:, 1:], y1[:, 1:])  # and no other output


# --------------------------------------------------- closed-form special cases

def test_matmul_integer_known_answer():
    M = K = N = 64
    i = np.arange(M * K)
    A = (i % 4).astype(np.float32)
    B = (np.arange(K * N) % 3).astype(np.float32)
    want = (A.reshape(M, K).astype(np.int64) @ B.reshape(K, N).astype(np.int64)).astype(np.float32).ravel()
    for nm, groups in (("matmul", (M * N + 63) // 64), ("matmul-tiled", (M // 16) * (N // 16)),
                       ("matmul-reg", ((M // 4) * (N // 4) + 63) // 64)):
        C = np.zeros(M * N, np.float32)
        orc.dispatch(nm, [A, B, C], [M, K, N], groups)
        assert np.array_equal(C, want), nm


def test_softmax_special_rows():
    N = 100
    a = np.zeros((3, N), np.float32)
    a[1] = np.linspace(-5, 5, N)
    a[2] = a[1] + 1000.0  # shift invariance after max subtraction
    a[2, ::3] = -1.0e30   # masked entries become exactly 0
    c = orc.softmax_rows(a.ravel(), 3, N).reshape(3, N)
    assert np.allclose(c[0], 1.0 / N, rtol=1e-6, atol=0)
    assert np.all(c[2, ::3] == 0.0)
    assert abs(c[1].sum() - 1.0) < 1e-5 and abs(c[2].sum() - 1.0) < 1e-5


def test_rope_tables_identity_and_inverse():
    rng = np.random.default_rng(5)
    seq, dim, heads = 4, 32, 2
    half = dim // heads // 2
    p = np.arange(seq)[:, None]
    th = p / 10000.0 ** (2.0 * np.arange(half)[None, :] / (2 * half))
    co, si = np.cos(th).astype(np.float32).ravel(), np.sin(th).astype(np.float32).ravel()
    x = rng.standard_normal(seq * dim).astype(np.float32)
    y = np.zeros_like(x)
    orc.dispatch("rope-apply", [x, co, si, np.array([1.0], np.float32), y], [seq, dim, heads], 1)
    assert np.array_equal(y[:dim], x[:dim])  # position 0 is the identity
    z = np.zeros_like(x)
    orc.dispatch("rope-apply", [y, co, si, np.array([-1.0], np.float32), z], [seq, dim, heads], 1)
    assert np.allclose(z, x, atol=1e-6)      # sign -1 undoes sign +1 (kernels.el:853-856)
    # rotation preserves each pair's norm
    n0 = (x.reshape(-1, 2) ** 2).sum(1)
    n1 = (y.reshape(-1, 2) ** 2).sum(1)
    assert np.allclose(n0, n1, rtol=1e-5)


def test_decode_attention_position_zero_is_v_row_zero():
    rng = np.random.default_rng(9)
    dim, heads, kvh, maxseq, hd = 128, 2, 1, 8, 64
    q = rng.standard_normal(dim).astype(np.float32)
    ck = rng.standard_normal(maxseq * kvh * hd).astype(np.float32)
    cv = rng.standard_normal(maxseq * kvh * hd).astype(np.float32)
    c = np.zeros(dim, np.float32)
    orc.dispatch("decode-attn", [q, ck, cv, np.array([0.0], np.float32), c], [dim, heads, kvh], 2)
    assert np.array_equal(c, np.tile(cv[:hd], heads))
    # causal prefill: query 0 attends only key 0
    seq = 5
    Q = rng.standard_normal(seq * heads * hd).astype(np.float32)
    K = rng.standard_normal(seq * kvh * hd).astype(np.float32)
    V = rng.standard_normal(seq * kvh * hd).astype(np.float32)
    ctx = np.zeros(seq * heads * hd, np.float32)
    orc.dispatch("attn-causal-gqa", [Q, K, V, ctx], [seq, heads, kvh, hd], 1)
    assert np.array_equal(ctx[:hd], V[:hd]) and np.array_equal(ctx[hd:2 * hd], V[:hd])


def test_scores_softmax_context_compose_to_fused_attention():
    rng = np.random.default_rng(21)
    seq, heads, kvh, hd = 7, 4, 2, 16
    dim = heads * hd
    Q = rng.standard_normal(seq * dim).astype(np.float32)
    K = rng.standard_normal(seq * kvh * hd).astype(np.float32)
    V = rng.standard_normal(seq * kvh * hd).astype(np.float32)
    S = np.zeros(heads * seq * seq, np.float32)
    orc.dispatch("attn-scores", [Q, K, S], [seq, dim, heads, kvh], 10)
    P = orc.softmax_rows(S, heads * seq, seq)
    C1 = np.zeros(seq * dim, np.float32)
    orc.dispatch("attn-context", [P, V, C1], [seq, dim, heads, kvh], 10)
    C2 = np.zeros(seq * dim, np.float32)
    orc.dispatch("attn-causal-gqa", [Q, K, V, C2], [seq, heads, kvh, hd], 1)
    assert np.max(np.abs(C1 - C2)) < 1e-5


def test_robust_access_never_faults_the_checker():
    # a POS far past the cache and a token past the table read zeros
    c = np.zeros(8, np.float32)
    orc.dispatch("cache-append", [np.ones(4, np.float32), np.array([1e9], np.float32), c], [4], 1)
    assert not c.any()
    out = np.full(4, 7, np.float32)
    orc.dispatch("embed-gather", [np.array([99.0], np.float32), np.ones(8, np.float32), out], [1, 4], 1)
    assert not out.any()


def test_transposed_linear_adjoint_identity():
    """ternary-rows and ternary-rows-t are adjoint: <W x, g> = <x, W' g>
    (test/ternary-kernel-test.el:130-145), with the block scales
    load-bearing (a different scale per (row, block))."""
    rng = np.random.default_rng(20260921)
    seq, out, cols, nblk = 3, 6, 256, 2
    wng = (cols + 15) // 16
    w = rng.integers(0, 2 ** 32, out * wng, dtype=np.uint64).astype(np.uint32).view(np.float32)
    beta = (np.abs(rng.standard_normal(out * nblk)) * 0.05 + 0.01).astype(np.float32)
    x = rng.standard_normal(seq * cols).astype(np.float32)
    g = rng.standard_normal(seq * out).astype(np.float32)
    y = np.zeros(seq * out, np.float32)
    orc.dispatch("ternary-rows", [x, w, np.zeros(out, np.float32), beta, y], [seq, out, cols, nblk, wng],
                 (seq * out + 63) // 64)
    xt = np.zeros(seq * cols, np.float32)
    orc.dispatch("ternary-rows-t", [w, beta, g, xt], [out, cols, nblk, wng, seq], (seq * cols + 63) // 64)
    left = float(np.dot(y.astype(np.float64), g))
    right = float(np.dot(x.astype(np.float64), xt))
    assert abs(left - right) <= 1e-5 * max(1e-6, abs(left))
