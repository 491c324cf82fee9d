"""CPU compositions of the reference kernels that the decoder-layer fusions
replace, built from the oracle's restatements (test infrastructure only).

Each helper chains the oracle's statements of the named DSL kernels in the
order a reference caller would dispatch them:
  linear      pack-act-rows (kernels.el:884-932) + bitlinear-dp4a-1f on the
              2-bit weights unpacked to int8 lanes (kernels.el:619-634)
  rms         rmsnorm-istd + rmsnorm-fwd (kernels.el:1249-1265), eps a parameter
  rope_b      decode-rope-b (kernels.el:340-355)
  silu_mul    silu-mul (kernels.el:186-193)
  attention   decode-attn-b (kernels.el:366-390) over fp16 caches
and RefStack runs the decoder stack's token step from those pieces.
"""
import numpy as np

import nlg_oracle as orc

f32 = np.float32


def linear(x, w2, beta, seq, out, cols, bias=None, per_row=False):
    xq, g = orc.pack_act_rows(np.ascontiguousarray(x, f32), seq, cols)
    return orc.ternary_linear_i8(xq, g, w2, bias, beta, seq, out, cols, beta_per_row=per_row)


def rms(x, gain, eps, rows, cols):
    return orc.rmsnorm_rows(x, gain, eps, rows, cols)


def silu_mul(a, b):
    a = np.ascontiguousarray(a, f32).copy()
    b = np.ascontiguousarray(b, f32).copy()
    c = np.zeros(a.size, f32)
    orc.dispatch("silu-mul", [a, b, c], [a.size], (a.size + 63) // 64)
    return c


def rope_b(x, co, si, pos, B, cols, heads):
    x = np.ascontiguousarray(x, f32).copy()
    c = np.zeros(B * cols, f32)
    npairs = B * cols // 2
    orc.dispatch("decode-rope-b", [x, np.ascontiguousarray(co, f32), np.ascontiguousarray(si, f32),
                                   np.array([1.0], f32), np.array([float(pos)], f32), c],
                 [B, cols, heads], (npairs + 63) // 64)
    return c


class RefStack:
    """The decoder stack's step (nelisp-gpu_amd/csrc/nlg_stack.hip) composed
    from the reference kernels, with weights downloaded from a device stack.
    seqs picks which of the device batch's sequences it follows (all by
    default); sequences are independent, so a subset steps exactly as the
    whole batch would."""

    def __init__(self, stack, seqs=None):
        c = stack.cfg
        self.c = c
        self.seqs = list(range(c.batch)) if seqs is None else list(seqs)
        self.nq, self.nkv = c.heads * c.head_dim, c.kv_heads * c.head_dim
        g = stack.tensor
        self.L = []
        for l in range(c.layers):
            self.L.append({
                "wqkv": g("wqkv", l, np.uint32), "bqkv": g("bqkv", l), "wo": g("wo", l, np.uint32),
                "bo": g("bo", l), "wgu": g("wgu", l, np.uint32), "bgu": g("bgu", l),
                "wd": g("wd", l, np.uint32), "bd": g("bd", l), "gattn": g("gattn", l),
                "gffn": g("gffn", l),
            })
        self.wlm, self.blm, self.gfinal = g("wlm", -1, np.uint32), g("blm"), g("gfinal")
        self.emb = g("emb").reshape(c.vocab, c.d_model)
        self.co, self.si = g("rope_cos"), g("rope_sin")
        shape = (len(self.seqs), c.kv_heads, c.max_seq, c.head_dim)
        self.kc = [np.zeros(shape, np.float16) for _ in range(c.layers)]
        self.vc = [np.zeros(shape, np.float16) for _ in range(c.layers)]

    def load_caches(self, stack, upto, layers=None):
        """Take the device stack's fp16 K/V rows of positions < upto (e.g.
        after a prefill) as this composition's own, so the next step starts
        from the same state (every layer, or the given ones)."""
        c = self.c
        for l in (range(c.layers) if layers is None else layers):
            for name, dst in (("kc", self.kc[l]), ("vc", self.vc[l])):
                dev = stack.tensor(name, l, np.float16).reshape(c.batch, c.kv_heads, c.max_seq, c.head_dim)
                dst[:] = 0
                dst[:, :, :upto] = dev[self.seqs, :, :upto]

    def layer(self, l, x, pos):
        """Layer l on the residual stream x [len(seqs) x d_model] at position
        pos: appends this position's K/V to layer l's caches and returns the
        stream after the layer."""
        c, B, d, f = self.c, len(self.seqs), self.c.d_model, self.c.d_ff
        nq, nkv, hd = self.nq, self.nkv, c.head_dim
        w = self.L[l]
        x = np.ascontiguousarray(x, f32).ravel()
        xn = rms(x, w["gattn"], c.rms_eps, B, d)
        qkv = linear(xn, w["wqkv"], w["bqkv"], B, nq + 2 * nkv, d, per_row=True).reshape(B, -1)
        q = rope_b(qkv[:, :nq].ravel(), self.co, self.si, pos, B, nq, c.heads)
        k = rope_b(qkv[:, nq:nq + nkv].ravel(), self.co, self.si, pos, B, nkv, c.kv_heads)
        v = qkv[:, nq + nkv:]
        self.kc[l][:, :, pos, :] = k.reshape(B, c.kv_heads, hd).astype(np.float16)
        self.vc[l][:, :, pos, :] = v.reshape(B, c.kv_heads, hd).astype(np.float16)
        att = orc.decode_attn_f16(q, self.kc[l].view(np.uint16), self.vc[l].view(np.uint16), pos,
                                  B, c.heads, c.kv_heads, hd, c.max_seq)
        x = (x + linear(att, w["wo"], w["bo"], B, d, nq)).astype(f32)
        xn = rms(x, w["gffn"], c.rms_eps, B, d)
        gu = linear(xn, w["wgu"], w["bgu"], B, 2 * f, d, per_row=True).reshape(B, 2 * f)
        h = silu_mul(gu[:, 0::2].ravel(), gu[:, 1::2].ravel())
        return (x + linear(h, w["wd"], w["bd"], B, d, f)).astype(f32).reshape(B, d)

    def head(self, x):
        """Final RMSNorm and the LM head: logits [len(seqs) x vocab]."""
        c, B = self.c, len(self.seqs)
        xn = rms(np.ascontiguousarray(x, f32).ravel(), self.gfinal, c.rms_eps, B, c.d_model)
        return linear(xn, self.wlm, self.blm, B, c.vocab, c.d_model).reshape(B, c.vocab)

    def embed(self, tokens):
        return self.emb[np.asarray(tokens)].astype(f32).reshape(len(self.seqs), self.c.d_model)

    def step(self, tokens, pos):
        """One token per followed sequence at position pos; returns their
        logits [len(seqs) x vocab]."""
        x = self.embed(tokens)
        for l in range(self.c.layers):
            x = self.layer(l, x, pos)
        return self.head(x)
