"""fp16 attention never lets a cache row it does not attend reach its output.

The reference's attention kernels read only the rows of positions 0..pos
(decode-attn, kernels.el:366-390; the paged, ring and prompt forms likewise),
so whatever a caller's cache holds past them -- unwritten memory, a previous
sequence's rows, NaN or infinity bit patterns -- cannot change the result.
The kernels here fetch whole position blocks, and some fetch them before the
position is known; every such row must be zeroed or masked before it meets a
probability, because 0 x NaN and 0 x Inf are NaN.  Each test fills every row
past the attended range with NaN / +Inf / -Inf and compares with the CPU
restatement (which never reads them), at the shapes that select each code
path: the VALU and matrix-core chunk passes, plain and non-temporal loads,
the per-head B=1 pass, paged pools, ring caches before they fill, and the
prompt attention's last, partly valid key block.
"""
import numpy as np
import pytest

import nlg_oracle as orc
import nlgpu

pytestmark = pytest.mark.gpu
f32 = np.float32
JUNK = np.array([0x7E00, 0x7C00, 0xFC00], np.uint16)  # NaN, +Inf, -Inf


@pytest.fixture(scope="module", autouse=True)
def device():
    nlgpu.init()
    yield


def poison_rows(c, B, kvh, rows, hd, first):
    """Rows first[b].. of sequence b's every kv head set to NaN / +-Inf bits."""
    c = c.reshape(B, kvh, rows, hd).copy()
    for b in range(B):
        n = rows - first[b]
        if n > 0:
            c[b, :, first[b]:, :] = JUNK[np.arange(n) % 3][None, :, None]
    return c.ravel()


def check(got, want, bar):
    assert np.isfinite(got).all(), f"{np.count_nonzero(~np.isfinite(got))} non-finite outputs"
    err = np.abs(got - want).max() / np.abs(want).max()
    print(f"  max err / max|out| = {err:.2e}", flush=True)
    assert err <= bar


@pytest.mark.parametrize("B,heads,kvh,hd,max_seq,positions", [
    (3, 8, 8, 64, 130, [0, 77, 128]),              # VALU chunk pass, plain loads
    (1, 20, 5, 128, 768, [0, 200, 700]),           # one query head per workgroup (B=1)
    (16, 20, 5, 128, 400, [0, 31, 255, 300]),      # matrix-core chunk pass, plain loads
    (32, 20, 5, 128, 768, [31, 640])])             # matrix-core chunk pass, non-temporal loads
def test_decode_attention_ignores_rows_past_the_position(B, heads, kvh, hd, max_seq, positions):
    print(f"[gpu] unwritten rows: attention B={B} heads={heads}/{kvh} hd={hd} max_seq={max_seq}", flush=True)
    n = B * kvh * max_seq * hd
    k0 = nlgpu.normal(hd + 3 * B, n).astype(np.float16).view(np.uint16)
    v0 = nlgpu.normal(hd + 3 * B + 1, n).astype(np.float16).view(np.uint16)
    ws = nlgpu.DeviceArray(nlgpu.decode_attn_f16_workspace(B, heads, kvh, hd, max_seq))
    out = nlgpu.DeviceArray(B * heads * hd * 4)
    for pos in positions:
        print(f"  pos={pos}", flush=True)
        kc = poison_rows(k0, B, kvh, max_seq, hd, [pos + 1] * B)
        vc = poison_rows(v0, B, kvh, max_seq, hd, [pos + 1] * B)
        q = (nlgpu.normal(pos + 5, B * heads * hd) * f32(2.0)).astype(f32)
        nlgpu.decode_attn_f16(nlgpu.to_device(q), nlgpu.to_device(kc), nlgpu.to_device(vc),
                              nlgpu.to_device(np.array([pos], np.int32)), out, B, heads, kvh, hd, max_seq, ws)
        check(out.download(f32, B * heads * hd), orc.decode_attn_f16(q, kc, vc, pos, B, heads, kvh, hd, max_seq),
              2e-3)


@pytest.mark.parametrize("B,heads,kvh,hd,max_seq,P,pos0", [
    (2, 8, 2, 64, 130, 100, 30),      # the last key block partly past the prompt
    (1, 20, 5, 128, 768, 500, 0),     # the stack's shape, prompt not a multiple of 32
    (2, 4, 4, 64, 64, 33, 0)])
def test_prefill_attention_ignores_rows_past_the_prompt(B, heads, kvh, hd, max_seq, P, pos0):
    print(f"[gpu] unwritten rows: prefill B={B} heads={heads}/{kvh} hd={hd} P={P} pos0={pos0}", flush=True)
    n = B * kvh * max_seq * hd
    kc = poison_rows(nlgpu.normal(hd + 7, n).astype(np.float16).view(np.uint16), B, kvh, max_seq, hd, [pos0 + P] * B)
    vc = poison_rows(nlgpu.normal(hd + 8, n).astype(np.float16).view(np.uint16), B, kvh, max_seq, hd, [pos0 + P] * B)
    q = (nlgpu.normal(P + 9, B * P * heads * hd) * f32(2.0)).astype(f32)
    ctx = nlgpu.DeviceArray(B * P * heads * hd * 4)
    nlgpu.prefill_attn_f16(nlgpu.to_device(q), nlgpu.to_device(kc), nlgpu.to_device(vc),
                           nlgpu.to_device(np.array([pos0], np.int32)), B * P, P, heads, kvh, hd, max_seq, ctx)
    got = ctx.download(f32, B * P * heads * hd).reshape(B, P, heads * hd)
    qr = q.reshape(B, P, heads * hd)
    per = kvh * max_seq * hd
    assert np.isfinite(got).all(), f"{np.count_nonzero(~np.isfinite(got))} non-finite outputs"
    worst = 0.0
    for b in range(B):
        for i in range(P):
            want = orc.decode_attn_f16(qr[b, i], kc[b * per:(b + 1) * per], vc[b * per:(b + 1) * per], pos0 + i,
                                       1, heads, kvh, hd, max_seq)
            worst = max(worst, float(np.abs(got[b, i] - want).max() / np.abs(want).max()))
    print(f"  max err / max|out| = {worst:.2e}", flush=True)
    assert worst <= 1e-4


@pytest.mark.parametrize("B,heads,kvh,hd,nsink,win", [(3, 8, 1, 64, 0, 37), (4, 4, 4, 128, 4, 250),
                                                      (32, 20, 5, 128, 4, 764)])
def test_ring_attention_ignores_slots_not_yet_written(B, heads, kvh, hd, nsink, win):
    """Sequences whose stream has not filled the ring: slots past the
    position hold NaN / +-Inf."""
    print(f"[gpu] unwritten rows: ring B={B} heads={heads}/{kvh} hd={hd} nsink={nsink} win={win}", flush=True)
    cap = nsink + win
    rng = np.random.default_rng(B + win)
    pos = rng.integers(0, cap, B).astype(np.int32)
    pos[0] = 0
    pos[-1] = cap // 2
    first = [int(p) + 1 for p in pos]
    kc = poison_rows(nlgpu.normal(B + 21, B * kvh * cap * hd).astype(np.float16).view(np.uint16), B, kvh, cap, hd,
                     first)
    vc = poison_rows(nlgpu.normal(B + 22, B * kvh * cap * hd).astype(np.float16).view(np.uint16), B, kvh, cap, hd,
                     first)
    ang = np.outer(np.arange(cap), 1.0 / 500000.0 ** (np.arange(hd // 2) * 2.0 / hd))
    co, si = np.cos(ang).astype(f32), np.sin(ang).astype(f32)
    q = (nlgpu.normal(B + 23, B * heads * hd) * f32(2.0)).astype(f32)
    out = nlgpu.DeviceArray(B * heads * hd * 4)
    ws = nlgpu.DeviceArray(nlgpu.decode_attn_stream_f16_workspace(B, heads, kvh, hd, nsink, win))
    nlgpu.decode_attn_stream_f16(nlgpu.to_device(q), nlgpu.to_device(kc), nlgpu.to_device(vc), nlgpu.to_device(pos),
                                 nlgpu.to_device(co), nlgpu.to_device(si), out, B, heads, kvh, hd, nsink, win, ws)
    check(out.download(f32, B * heads * hd),
          orc.decode_attn_stream_f16(q, kc, vc, pos, co, si, B, heads, kvh, hd, nsink, win), 1e-4)


@pytest.mark.parametrize("B,heads,kvh,hd,bs,mbps,npool", [(4, 8, 2, 64, 7, 10, 60), (3, 20, 5, 128, 16, 48, 160),
                                                       (32, 20, 5, 128, 16, 48, 1600)])
def test_paged_attention_ignores_rows_past_each_length(B, heads, kvh, hd, bs, mbps, npool):
    """Pool rows no sequence attends (past its length in its last block, in
    blocks it has not reached, in blocks no table names) hold NaN / +-Inf."""
    print(f"[gpu] unwritten rows: paged B={B} heads={heads}/{kvh} hd={hd} bs={bs} mbps={mbps}", flush=True)
    rng = np.random.default_rng(B * 31 + hd)
    kvdim = kvh * hd
    table = rng.permutation(npool)[:B * mbps].reshape(B, mbps).astype(np.int32) if npool >= B * mbps else \
        rng.integers(0, npool, (B, mbps)).astype(np.int32)
    lens = rng.integers(0, bs * mbps, B).astype(np.int32)
    lens[0] = 0
    live = np.zeros(npool * bs, bool)
    for b in range(B):
        for p in range(int(lens[b]) + 1):
            live[table[b, p // bs] * bs + p % bs] = True
    kp = nlgpu.normal(B + 31, npool * bs * kvdim).astype(np.float16).view(np.uint16).reshape(npool * bs, kvdim)
    vp = nlgpu.normal(B + 32, npool * bs * kvdim).astype(np.float16).view(np.uint16).reshape(npool * bs, kvdim)
    dead = np.flatnonzero(~live)
    kp[dead] = JUNK[dead % 3][:, None]
    vp[dead] = JUNK[(dead + 1) % 3][:, None]
    kp, vp = kp.ravel(), vp.ravel()
    q = (nlgpu.normal(B + 33, B * heads * hd) * f32(2.0)).astype(f32)
    out = nlgpu.DeviceArray(B * heads * hd * 4)
    ws = nlgpu.DeviceArray(nlgpu.decode_attn_paged_f16_workspace(B, heads, kvh, hd, bs, mbps))
    nlgpu.decode_attn_paged_f16(nlgpu.to_device(q), nlgpu.to_device(kp), nlgpu.to_device(vp), nlgpu.to_device(lens),
                                nlgpu.to_device(table), npool, out, B, heads, kvh, hd, bs, mbps, ws)
    check(out.download(f32, B * heads * hd),
          orc.decode_attn_paged_f16(q, kp, vp, lens, table, npool, B, heads, kvh, hd, bs, mbps), 1e-4)
