"""The fused epilogues of the int8 matrix-core GEMM (128 tokens and more:
config 4 at B = 512 and every prefill) against the chained reference
kernels on the CPU (tests/layer_ref.py):

* SwiGLU  -- rmsnorm-istd/-fwd, pack-act-rows, bitlinear-dp4a-1f on the
  interleaved gate|up rows, silu-mul (kernels.el:1249-1265, :884-932,
  :619-634, :186-193);
* residual -- the linear then add2 (kernels.el:812-821), in place and not;
* QKV     -- the linear, decode-rope-b on q and k and cache-append-b of k
  and v into fp16 caches (kernels.el:340-365), for decode rows (row s =
  sequence s) and for prompt rows (row r = sequence r / qper at position
  pos0 + r % qper).

Each shape is chosen so the GEMM runs a given form: the wide-wave kernel
(k_tgemm_w: 256-row tiles, 4 waves of 64 rows x 64 tokens -- "w64" -- or x 32
tokens -- "w32"; activations staged by direct global-to-LDS loads), whose
cases cover every remainder of its six-chunk loop (1 to 10 chunks of 256
columns, 27) and ragged rows and tokens for both tile heights, the
small-batch kernel's single 10-chunk phase where it wins at 128+ tokens
("sb10"), or the wide-wave kernel's
32-token tiles with the columns split over 2, 3 or 4 slices for few tiles of
rows of 16+ chunks ("split": slices of 4..14 chunks, ragged rows and
tokens).  Every case runs twice: with the weights' row layout, then with a
registered tiled copy of them (nlg_ternary_tiled_register), which must give
the same bits.  The
activations of the RMSNorm cases are small integers, so the sum of squares
is exact in any order and everything but SiLU's exp is bit-exact; SwiGLU's
gate uses the device exp and is held to 1e-5 relative (the north star's
bar is 1e-4).
"""
import numpy as np
import pytest

import layer_ref as ref
import nlgpu

pytestmark = pytest.mark.gpu
f32 = np.float32


@pytest.fixture(scope="module", autouse=True)
def device():
    nlgpu.init()
    yield


def int_rows(seed, n):
    """Integer activations in [-3, 3]: every partial sum of squares is exact."""
    return (nlgpu.trits(seed, (n,)).astype(f32) * f32(3) - nlgpu.trits(seed + 1, (n,)).astype(f32)).astype(f32)


def weights(seed, out, cols, per_row):
    w2 = nlgpu.pack_ternary(nlgpu.trits(seed, (out, cols)))
    beta = (f32(0.5) + nlgpu.uniform(seed + 1, out if per_row else 1).astype(f32)) / f32(np.sqrt(cols))
    return w2, beta.astype(f32)


def gains(seed, n):
    return (f32(0.75) + f32(0.5) * nlgpu.uniform(seed, n).astype(f32)).astype(f32)


def same_bits(a, b, what=""):
    a, b = np.asarray(a, f32).ravel(), np.asarray(b, f32).ravel()
    bad = np.flatnonzero(a.view(np.uint32) != b.view(np.uint32))
    assert bad.size == 0, f"{what}: {bad.size} differ, first {bad[:4]}: {a[bad[:3]]} vs {b[bad[:3]]}"


def with_tiled_copy(dw, rows, cols, run):
    """run() again with a tiled copy of dw registered, then drop the copy."""
    nlgpu.ternary_tiled_register(dw, rows, cols)
    try:
        return run()
    finally:
        nlgpu.ternary_tiled_unregister(dw)


def row_tile(seq, out, cols):
    """The batched GEMM's form for seq >= 128 tokens, or 65+ tokens over more
    than 512 64-row x 32-token tiles, either weight layout (nlg_tgemm.hip's
    choice): "small" -- the small-batch kernels, below 65 tokens or 513
    tiles; "sb10" -- the small-batch kernel's single 10-chunk phase, for
    rows of 9..10 chunks over 128..256 such tiles; "split" -- 32-token tiles
    with the columns split over gridDim.z slices, for at most 170 256-row
    tiles of rows of 16+ chunks -- else 256-row tiles of 64 tokens ("w64",
    once there are 400 of them) or 32 ("w32")."""
    rt = (out + 255) // 256
    t1, t2 = rt * ((seq + 31) // 32), rt * ((seq + 63) // 64)
    t64x32 = (out + 63) // 64 * ((seq + 31) // 32)
    if seq < 128 and (seq <= 64 or t64x32 <= 512):
        return "small"
    if 8 < cols // 256 <= 10 and 128 <= t64x32 <= 256:
        return "sb10"
    if cols // 256 >= 16 and t1 <= 170:
        return "split"
    return "w64" if t2 >= 400 else "w32"


SWIGLU = [(128, 6912, 2560, True, "w32"), (512, 6912, 2560, True, "w64"), (600, 6912, 2560, True, "w64"),
          (512, 640, 4096, False, "split"), (400, 4096, 1024, True, "w32"), (128, 1280, 2560, True, "sb10"), (512, 3072, 1024, True, "w32"),
          (300, 3840, 2560, False, "w32"),
          (1200, 6144, 1024, True, "w64"),   # 4 chunks
          (1100, 4096, 1536, False, "w64"),  # 6 chunks: one whole group
          (96, 6912, 2560, True, "w32"), (72, 6912, 1280, False, "w32")]  # 65+ tokens, 648 64-row tiles


@pytest.mark.parametrize("seq,dff,cols,rms,tile", SWIGLU)
def test_batched_swiglu(seq, dff, cols, rms, tile):
    assert row_tile(seq, 2 * dff, cols) == tile
    print(f"[gpu] batched swiglu seq={seq} dff={dff} cols={cols} rms={rms} tile={tile}", flush=True)
    x = int_rows(dff + seq, seq * cols) if rms else nlgpu.normal(dff + seq, seq * cols)
    g = gains(cols + 2, cols)
    w2, beta = weights(dff + 11, 2 * dff, cols, per_row=True)
    dh = nlgpu.DeviceArray(seq * dff * 4)
    dx, dg, dw, db = nlgpu.to_device(x), nlgpu.to_device(g) if rms else None, nlgpu.to_device(w2), nlgpu.to_device(beta)

    def run():
        dh.zero()
        nlgpu.rms_ternary_swiglu(dx, dg, 1e-5, dw, db, dh, seq, dff, cols)
        return dh.download(f32, seq * dff)

    got = run()
    xn = ref.rms(x, g, 1e-5, seq, cols) if rms else x
    gu = ref.linear(xn, w2, beta, seq, 2 * dff, cols, per_row=True).reshape(seq, 2 * dff)
    want = ref.silu_mul(gu[:, 0::2].ravel(), gu[:, 1::2].ravel())
    err = np.abs(got - want)
    print(f"  max rel err {np.max(err / np.maximum(np.abs(want), 1e-30)):.2e}", flush=True)
    assert np.all(err <= 1e-5 * np.abs(want) + 1e-7 * np.abs(want).max())
    same_bits(with_tiled_copy(dw, 2 * dff, cols, run), got, "tiled copy")


RESID = [(128, 2560, 6912, "split"), (512, 2560, 6912, "split"), (384, 2560, 6912, "split"),  # 4, 3, 2 slices
         (200, 1000, 4352, "split"),                          # 4 slices of 4..5 chunks, ragged rows and tokens
         (100, 9000, 6912, "split"),                          # 100 tokens over 564 64-row tiles: 3 slices, ragged
         (160, 2560, 2560, "sb10"), (150, 2500, 2304, "sb10"),  # one 10- / 9-chunk phase, ragged
         (1024, 2560, 6912, "w32"), (512, 8192, 2560, "w32"), (600, 13824, 2560, "w64"),
         (200, 1000, 512, "w32"), (512, 6144, 2560, "w32"), (512, 2560, 2560, "w32"),
         (128, 2048, 256, "w32"), (256, 2048, 1536, "w32"), (300, 13800, 768, "w32"),  # 1, 6, 3 chunks
         (512, 8192, 1280, "w32"),                                                      # 5 chunks
         (4096, 2048, 256, "w64"), (4096, 2048, 768, "w64"),  # 1 and 3 chunks
         (4100, 2000, 1280, "w64"),                            # 5 chunks, ragged rows and tokens
         (2700, 3000, 1792, "w64")]                            # 7 chunks: a group and one more


_RESID_WANT = {}  # the last shape's reference (the in-place case follows the other)


@pytest.mark.parametrize("inplace", [False, True])
@pytest.mark.parametrize("seq,out,cols,tile", RESID)
def test_batched_residual(seq, out, cols, tile, inplace):
    assert row_tile(seq, out, cols) == tile
    print(f"[gpu] batched residual seq={seq} out={out} cols={cols} tile={tile} inplace={inplace}", flush=True)
    x, res = nlgpu.normal(cols + seq, seq * cols), nlgpu.normal(out + seq, seq * out)
    w2, beta = weights(cols + out, out, cols, per_row=bool(out % 3))
    bias = (nlgpu.normal(out + 1, out) * f32(0.1)).astype(f32)
    dres = nlgpu.to_device(res)
    dy = dres if inplace else nlgpu.DeviceArray(seq * out * 4)
    dx, dw, dbias, db = nlgpu.to_device(x), nlgpu.to_device(w2), nlgpu.to_device(bias), nlgpu.to_device(beta)

    def run():
        dres.upload(res)
        if not inplace:
            dy.zero()
        nlgpu.ternary_linear_residual(dx, dw, dbias, db, dres, dy, seq, out, cols, beta_per_row=bool(out % 3))
        return dy.download(f32, seq * out)

    got = run()
    key = (seq, out, cols)
    if key not in _RESID_WANT:
        _RESID_WANT.clear()
        _RESID_WANT[key] = (res + ref.linear(x, w2, beta, seq, out, cols, bias=bias,
                                             per_row=bool(out % 3))).astype(f32)
    same_bits(got, _RESID_WANT[key], "residual")
    same_bits(with_tiled_copy(dw, out, cols, run), got, "tiled copy")


def rope_tables(max_seq, hd, theta=500000.0):
    half = hd // 2
    p = np.arange(max_seq)[:, None] / (theta ** (2.0 * np.arange(half)[None, :] / hd))
    return np.cos(p).astype(f32).ravel(), np.sin(p).astype(f32).ravel()


# rows, qper (0: decode rows), heads, kvheads, head_dim, cols, max_seq, pos0, tile
QKV = [(512, 512, 20, 5, 128, 2560, 768, 0, "w32"),     # config 5's prompt at B = 1
       (600, 200, 64, 16, 128, 2560, 256, 40, "w64"),   # three prompts
       (512, 256, 32, 8, 128, 2560, 320, 40, "w32"),    # two prompts
       (512, 128, 64, 32, 128, 2560, 160, 20, "w64"),   # four prompts
       (128, 64, 8, 2, 64, 1024, 100, 50, "w32"),       # positions run past max_seq: no cache store there
       (128, 0, 20, 5, 128, 2560, 16, 5, "sb10"),       # 128 decode rows at one position
       (128, 0, 8, 2, 128, 4096, 16, 5, "split"),       # the same, rows of 16 chunks
       (256, 128, 8, 2, 128, 4352, 160, 20, "split"),   # two prompts, rows of 17 chunks
       (100, 0, 64, 16, 128, 2560, 16, 5, "w32"),       # 100 decode rows over 768 64-row tiles
       (2304, 256, 20, 5, 128, 2560, 320, 10, "w64"),   # nine prompts (10 chunks)
       (2304, 0, 20, 5, 128, 512, 8, 3, "w64")]         # 2304 decode rows (2 chunks)


@pytest.mark.parametrize("rows,qper,heads,kvh,hd,cols,max_seq,pos0,tile", QKV)
def test_batched_qkv_rope_append(rows, qper, heads, kvh, hd, cols, max_seq, pos0, tile):
    nq, nkv = heads * hd, kvh * hd
    out = nq + 2 * nkv
    assert row_tile(rows, out, cols) == tile
    print(f"[gpu] batched qkv rows={rows} qper={qper} heads={heads}/{kvh} hd={hd} pos0={pos0} tile={tile}",
          flush=True)
    nseq = rows // qper if qper else rows
    x, g = int_rows(cols + rows + pos0, rows * cols), gains(cols + 5, cols)
    w2, beta = weights(nq + pos0, out, cols, per_row=True)
    co, si = rope_tables(max_seq, hd)
    sentinel = np.full(nseq * kvh * max_seq * hd, 0x7BCD, np.uint16)
    dkc, dvc = nlgpu.to_device(sentinel), nlgpu.to_device(sentinel)
    dq = nlgpu.DeviceArray(rows * nq * 4)
    dw = nlgpu.to_device(w2)
    args = (nlgpu.to_device(x), nlgpu.to_device(g), 1e-5, dw, nlgpu.to_device(beta), dq, dkc,
            dvc, nlgpu.to_device(co), nlgpu.to_device(si), nlgpu.to_device(np.array([pos0], np.int32)))

    def run():
        dq.zero()
        dkc.upload(sentinel)
        dvc.upload(sentinel)
        if qper:
            nlgpu.rms_ternary_qkv_rope_prompt(*args, rows, qper, heads, kvh, hd, max_seq, cols)
        else:
            nlgpu.rms_ternary_qkv_rope(*args, rows, heads, kvh, hd, max_seq, cols)
        return (dq.download(f32, rows * nq).reshape(rows, nq),
                dkc.download(np.uint16).reshape(nseq, kvh, max_seq, hd),
                dvc.download(np.uint16).reshape(nseq, kvh, max_seq, hd))

    gq, kc, vc = run()
    tq, tk, tv = with_tiled_copy(dw, out, cols, run)
    same_bits(tq, gq, "tiled copy: q")
    assert np.array_equal(tk, kc) and np.array_equal(tv, vc), "tiled copy: caches"
    qkv = ref.linear(ref.rms(x, g, 1e-5, rows, cols), w2, beta, rows, out, cols, per_row=True).reshape(rows, -1)
    if not qper:  # every row at pos0: decode-rope-b over the whole batch at once
        q = ref.rope_b(qkv[:, :nq].ravel(), co, si, pos0, rows, nq, heads).reshape(rows, nq)
        k = ref.rope_b(qkv[:, nq:nq + nkv].ravel(), co, si, pos0, rows, nkv, kvh).reshape(rows, kvh, hd)
        same_bits(gq, q, "q")
        assert np.array_equal(kc[:, :, pos0], k.astype(np.float16).view(np.uint16))
        assert np.array_equal(vc[:, :, pos0], qkv[:, nq + nkv:].reshape(rows, kvh, hd).astype(np.float16).view(np.uint16))
        kc[:, :, pos0] = 0x7BCD
        vc[:, :, pos0] = 0x7BCD
    else:
        for r in range(rows):
            b, p = r // qper, pos0 + r % qper
            if p >= max_seq:
                continue  # q of such a row is unspecified; nothing may reach the caches
            q = ref.rope_b(qkv[r, :nq], co, si, p, 1, nq, heads)
            k = ref.rope_b(qkv[r, nq:nq + nkv], co, si, p, 1, nkv, kvh).reshape(kvh, hd)
            same_bits(gq[r], q, f"q row {r}")
            assert np.array_equal(kc[b, :, p], k.astype(np.float16).view(np.uint16)), r
            assert np.array_equal(vc[b, :, p], qkv[r, nq + nkv:].reshape(kvh, hd).astype(np.float16).view(np.uint16)), r
            kc[b, :, p] = 0x7BCD
            vc[b, :, p] = 0x7BCD
    assert np.all(kc == 0x7BCD) and np.all(vc == 0x7BCD)  # nothing else written


def test_qkv_prompt_rejects_ragged_rows():
    d = nlgpu.DeviceArray(1 << 16)
    pos = nlgpu.to_device(np.array([0], np.int32))
    with pytest.raises(nlgpu.NlgError, match="qper"):
        nlgpu.rms_ternary_qkv_rope_prompt(d, d, 1e-5, d, d, d, d, d, d, d, pos, 10, 4, 4, 2, 64, 16, 256)
    with pytest.raises(nlgpu.NlgError, match="qper"):
        nlgpu.rms_ternary_qkv_rope_prompt(d, d, 1e-5, d, d, d, d, d, d, d, pos, 10, 0, 4, 2, 64, 16, 256)


def test_tiled_copy_registration():
    """A registered tiled copy follows every write the library makes into its
    weights (nlg_upload, nlg_copy_d2d, nlg_zero, a repack): calls at 1 token
    (the GEMV, row layout), 8 tokens (the small-batch GEMM) and 512 tokens
    (the 128 x 128 tiles) all give the oracle's bits for the new weights.
    Registering again refreshes it too; after unregistering, the row layout
    is read.  Shapes the copy cannot serve are refused or read the rows."""
    out, cols = 512, 1024
    seqs = (1, 8, 512)
    xs = {n: nlgpu.normal(7 + n, n * cols) for n in seqs}
    dxs = {n: nlgpu.to_device(xs[n]) for n in seqs}
    w_a, beta = weights(31, out, cols, per_row=False)
    w_b, _ = weights(32, out, cols, per_row=False)
    dw, db = nlgpu.to_device(w_a), nlgpu.to_device(beta)
    dy = nlgpu.DeviceArray(max(seqs) * out * 4)

    def check(w, what):
        for n in seqs:
            dy.zero()
            nlgpu.ternary_linear(dxs[n], dw, None, db, dy, n, out, cols)
            same_bits(dy.download(f32, n * out), ref.linear(xs[n], w, beta, n, out, cols), f"{what}, {n} tokens")

    nlgpu.ternary_tiled_register(dw, out, cols)
    try:
        check(w_a, "tiled copy of A")
        dw.upload(w_b)
        check(w_b, "after nlg_upload of B")
        da = nlgpu.to_device(w_a)
        _check_rc(nlgpu.lib().nlg_copy_d2d(dw.ptr, da.ptr, w_a.nbytes, None))
        check(w_a, "after nlg_copy_d2d of A")
        dw.upload(w_b[:out // 2], offset=0)  # a partial write: the first half of the rows
        w_mix = np.concatenate([w_b[:out // 2], w_a[out // 2:]])
        check(w_mix, "after a partial upload")
        dw.zero()
        check(np.zeros_like(w_a), "after nlg_zero")
        # a repack writing into the registered buffer (int8 lanes of B -> 2-bit)
        lanes = nlgpu.unpack_ternary(w_b, cols).astype(np.int8).reshape(out, cols).view(np.uint32)
        dl = nlgpu.to_device(np.ascontiguousarray(lanes))
        nlgpu.repack_i8_to_2bit(dl, out, cols, dw)
        check(w_b, "after a repack into it")
        nlgpu.ternary_tiled_register(dw, out, cols)  # again: a refresh in place
        check(w_b, "registered again")
        # another shape over the same pointer is not served by the copy
        dy.zero()
        nlgpu.ternary_linear(dxs[512], dw, None, db, dy, 512, out - 32, cols)
        same_bits(dy.download(f32, 512 * (out - 32)), ref.linear(xs[512], w_b[:out - 32], beta, 512, out - 32, cols),
                  "other rows: row layout")
    finally:
        nlgpu.ternary_tiled_unregister(dw)
    dw.upload(w_a)
    check(w_a, "unregistered: row layout")
    nlgpu.ternary_tiled_unregister(dw)  # no copy: a no-op
    with pytest.raises(nlgpu.NlgError, match="multiple of 256"):
        nlgpu.ternary_tiled_register(dw, out, 1000)


def _check_rc(rc):
    if rc:
        raise nlgpu.NlgError(nlgpu.last_error())


def test_tiled_copy_dropped_with_its_memory():
    """nlg_free of registered weights drops the registration: new weights in
    a buffer allocated afterwards -- at the same address, which the
    allocator hands back for the same size -- are read as they are, not
    through the freed buffer's copy."""
    out, cols, n = 512, 1024, 512
    x = nlgpu.normal(9, n * cols)
    w_a, beta = weights(41, out, cols, per_row=False)
    w_b, _ = weights(42, out, cols, per_row=False)
    dx, db, dy = nlgpu.to_device(x), nlgpu.to_device(beta), nlgpu.DeviceArray(n * out * 4)
    reused = 0
    for attempt in range(4):
        d1 = nlgpu.to_device(w_a)
        nlgpu.ternary_tiled_register(d1, out, cols)
        nlgpu.ternary_linear(dx, d1, None, db, dy, n, out, cols)
        same_bits(dy.download(f32, n * out), ref.linear(x, w_a, beta, n, out, cols), "registered A")
        addr = d1.ptr
        d1.free()  # no unregister: nlg_free drops it
        d2 = nlgpu.to_device(w_b)
        reused += d2.ptr == addr
        dy.zero()
        nlgpu.ternary_linear(dx, d2, None, db, dy, n, out, cols)
        same_bits(dy.download(f32, n * out), ref.linear(x, w_b, beta, n, out, cols), f"new buffer, attempt {attempt}")
        d2.free()
    print(f"  same address handed back in {reused} of 4 attempts", flush=True)


# 4..127 tokens (at 65+, up to 512 64-row x 32-token tiles): the 16x16x64 GEMM
# with 64-row workgroups (many rows) or the 16-row column-split form (few rows),
# each on the row layout and on a tiled copy
SMALL = [(8, 13824, 2560), (32, 13824, 2560), (100, 6912, 1024), (32, 2560, 6912), (16, 3840, 2560),
         (32, 2560, 2560), (77, 1000, 512)]


@pytest.mark.parametrize("seq,out,cols", SMALL)
def test_small_batch_tiled_copy(seq, out, cols):
    assert row_tile(seq, out, cols) == "small"
    print(f"[gpu] small batch seq={seq} out={out} cols={cols}", flush=True)
    x, res = nlgpu.normal(cols + seq + 1, seq * cols), nlgpu.normal(out + seq + 1, seq * out)
    w2, beta = weights(cols + out + 1, out, cols, per_row=True)
    bias = (nlgpu.normal(out + 2, out) * f32(0.1)).astype(f32)
    dx, dw, dbias, db = nlgpu.to_device(x), nlgpu.to_device(w2), nlgpu.to_device(bias), nlgpu.to_device(beta)
    dres, dy = nlgpu.to_device(res), nlgpu.DeviceArray(seq * out * 4)

    def run():
        dy.zero()
        nlgpu.ternary_linear_residual(dx, dw, dbias, db, dres, dy, seq, out, cols, beta_per_row=True)
        return dy.download(f32, seq * out)

    got = run()
    want = (res + ref.linear(x, w2, beta, seq, out, cols, bias=bias, per_row=True)).astype(f32)
    same_bits(got, want, "residual")
    same_bits(with_tiled_copy(dw, out, cols, run), got, "tiled copy")
