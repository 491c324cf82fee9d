"""Python binding of libnlgpu, the MI355X implementation of nelisp-gpu's
quantized-LLM kernel path.

This is a thin ctypes layer over the C ABI in include/nlgpu.h: device
buffers, kernels by reference name (`dispatch`), the typed hot path
(`pack_act_rows`, `ternary_linear_i8`, `softmax_rows`), events and graphs.
It loads the in-tree ``lib/libnlgpu.so`` and raises if it is missing -- there
is no CPU fallback anywhere in this module.

It also holds the data-format helpers a caller needs: packing ternary
weights into the reference's 2-bit layout (test/ternary-kernel-test.el:40-50,
lisp/nelisp-gpu-kernels.el:700-746) and a seeded counter-based generator
(SplitMix64) for reproducible synthetic inputs.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Iterable, Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libnlgpu.so")
BIN_DIR = os.path.join(HERE, "bin")


class NlgError(RuntimeError):
    pass


class Buffer(C.Structure):
    _fields_ = [("ptr", C.c_void_p), ("nfloats", C.c_uint32)]


class StackConfig(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("layers", "d_model", "heads", "kv_heads", "head_dim",
                                          "d_ff", "vocab", "max_seq", "batch")] + \
               [("rms_eps", C.c_float), ("rope_theta", C.c_float), ("seed", C.c_uint64)]


_lib = None


def lib() -> C.CDLL:
    """The loaded libnlgpu (raises NlgError if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise NlgError(f"{LIB_PATH} is missing: build it first (python -c "
                       f"'import __graft_entry__; __graft_entry__.build()')")
    L = C.CDLL(LIB_PATH)
    vp, u32, i32, sz = C.c_void_p, C.c_uint32, C.c_int, C.c_size_t
    f32p, u32p = C.POINTER(C.c_float), C.POINTER(C.c_uint32)
    sigs = {
        "nlg_init": (i32, [i32]),
        "nlg_shutdown": (i32, []),
        "nlg_last_error": (C.c_char_p, []),
        "nlg_device_name": (i32, [C.c_char_p, sz]),
        "nlg_device_info": (i32, [C.POINTER(i32), C.c_char_p, sz]),
        "nlg_malloc": (vp, [sz]),
        "nlg_free": (i32, [vp]),
        "nlg_upload": (i32, [vp, vp, sz]),
        "nlg_download": (i32, [vp, vp, sz]),
        "nlg_copy_d2d": (i32, [vp, vp, sz, vp]),
        "nlg_zero": (i32, [vp, sz, vp]),
        "nlg_upload_file": (i32, [vp, C.c_char_p, C.c_uint64, sz, C.POINTER(sz)]),
        "nlg_stream_create": (vp, []),
        "nlg_stream_destroy": (i32, [vp]),
        "nlg_stream_sync": (i32, [vp]),
        "nlg_default_stream": (vp, []),
        "nlg_event_create": (vp, []),
        "nlg_event_destroy": (i32, [vp]),
        "nlg_event_record": (i32, [vp, vp]),
        "nlg_event_elapsed_ms": (i32, [vp, vp, C.POINTER(C.c_float)]),
        "nlg_kernel_count": (i32, []),
        "nlg_kernel_name": (C.c_char_p, [i32]),
        "nlg_kernel_lookup": (i32, [C.c_char_p]),
        "nlg_kernel_abi": (i32, [C.c_char_p, C.POINTER(u32), C.POINTER(u32)]),
        "nlg_dispatch": (i32, [C.c_char_p, C.POINTER(Buffer), u32, C.POINTER(u32), u32, u32, vp]),
        "nlg_graph_begin": (i32, [vp]),
        "nlg_graph_end": (i32, [vp, C.POINTER(vp)]),
        "nlg_graph_launch": (i32, [vp, vp]),
        "nlg_graph_destroy": (i32, [vp]),
        "nlg_pack_act_rows": (i32, [vp, vp, vp, u32, u32, vp]),
        "nlg_ternary_linear_i8": (i32, [vp, vp, vp, vp, vp, i32, vp, u32, u32, u32, vp]),
        "nlg_ternary_linear_i8_cfg": (i32, [vp, vp, vp, vp, vp, i32, vp, u32, u32, u32, i32, i32, vp]),
        "nlg_softmax_rows": (i32, [vp, vp, u32, u32, vp]),
        "nlg_ternary_linear": (i32, [vp, vp, vp, vp, i32, vp, vp, u32, u32, u32, vp, sz, vp]),
        "nlg_ternary_linear_cfg": (i32, [vp, vp, vp, vp, i32, vp, vp, u32, u32, u32, i32, vp, sz, vp]),
        "nlg_ternary_linear_workspace": (sz, [u32, u32]),
        "nlg_ternary_linear_noalloc": (i32, [vp, vp, vp, vp, i32, vp, vp, u32, u32, u32, vp]),
        "nlg_rms_ternary_linear": (i32, [vp, vp, C.c_float, vp, vp, vp, i32, vp, u32, u32, u32, vp]),
        "nlg_ternary_linear_residual": (i32, [vp, vp, vp, vp, i32, vp, vp, u32, u32, u32, vp]),
        "nlg_rms_ternary_swiglu": (i32, [vp, vp, C.c_float, vp, vp, i32, vp, u32, u32, u32, vp]),
        "nlg_rms_ternary_qkv_rope": (i32, [vp, vp, C.c_float, vp, vp, i32, vp, vp, vp, vp, vp, vp,
                                           u32, u32, u32, u32, u32, u32, vp]),
        "nlg_rms_ternary_qkv_rope_prompt": (i32, [vp, vp, C.c_float, vp, vp, i32, vp, vp, vp, vp, vp, vp,
                                                  u32, u32, u32, u32, u32, u32, u32, vp]),
        "nlg_rms_ternary_argmax": (i32, [vp, vp, C.c_float, vp, vp, i32, vp, vp, u32, u32, u32, vp,
                                         sz, vp]),
        "nlg_rms_ternary_argmax_workspace": (sz, [u32, u32]),
        "nlg_decode_attn_f16": (i32, [vp, vp, vp, vp, vp, u32, u32, u32, u32, u32, vp, sz, vp]),
        "nlg_decode_attn_f16_workspace": (sz, [u32, u32, u32, u32, u32]),
        "nlg_decode_attn_f16_chunks": (i32, [vp, vp, vp, vp, u32, u32, u32, u32, u32, vp, sz, vp]),
        "nlg_attn_ternary_linear_residual": (i32, [vp, sz, u32, u32, u32, u32, u32, vp, vp, vp, i32, vp,
                                                   vp, u32, vp]),
        "nlg_prefill_attn_f16": (i32, [vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, vp, vp]),
        "nlg_ternary_linear_timed": (i32, [vp, vp, vp, vp, u32, u32, vp, sz, vp]),
        "nlg_ternary_linear_timed_stamps": (sz, [u32]),
        "nlg_prefill_attn_ternary_linear_residual": (i32, [vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, vp, vp, vp,
                                                           vp, i32, vp, vp, u32, vp]),
        "nlg_repack_i8_to_2bit": (i32, [vp, u32, u32, vp, vp, vp]),
        "nlg_decode_attn_paged_f16": (i32, [vp, vp, vp, vp, vp, u32, vp, u32, u32, u32, u32, u32, u32, vp, sz,
                                            vp]),
        "nlg_decode_attn_paged_f16_workspace": (sz, [u32, u32, u32, u32, u32, u32]),
        "nlg_cache_append_paged_f16": (i32, [vp, vp, vp, u32, vp, u32, u32, u32, u32, vp]),
        "nlg_decode_attn_stream_f16": (i32, [vp, vp, vp, vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, vp, sz,
                                             vp]),
        "nlg_decode_attn_stream_f16_workspace": (sz, [u32, u32, u32, u32, u32, u32]),
        "nlg_cache_append_ring_f16": (i32, [vp, vp, vp, u32, u32, u32, u32, u32, vp]),
        "nlg_attn_entries_f16": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, u32, vp, sz,
                                       vp]),
        "nlg_attn_entries_f16_workspace": (sz, [u32, u32, u32, u32, u32]),
        "nlg_block_copy_f16": (i32, [vp, vp, vp, u32, u32, u32, u32, vp]),
        "nlg_repack_packed_to_2bit": (i32, [vp, u32, u32, u32, u32, vp, vp, vp]),
        "nlg_ternary_tiled_register": (i32, [vp, u32, u32, vp]),
        "nlg_ternary_tiled_unregister": (i32, [vp]),
        "nlg_fill_normal": (i32, [vp, C.c_uint64, C.c_uint64, C.c_float, u32, vp]),
        "nlg_stack_create": (i32, [C.POINTER(StackConfig), C.POINTER(vp)]),
        "nlg_stack_destroy": (None, [vp]),
        "nlg_stack_start": (i32, [vp, vp, u32]),
        "nlg_stack_prefill": (i32, [vp, vp, u32]),
        "nlg_stack_prefill_trace": (i32, [vp, vp, u32, vp]),
        "nlg_stack_step": (i32, [vp, u32, i32]),
        "nlg_stack_step_trace": (i32, [vp, vp]),
        "nlg_stack_position": (i32, [vp, C.POINTER(u32)]),
        "nlg_stack_tokens": (i32, [vp, vp, vp]),
        "nlg_stack_logits": (i32, [vp, vp]),
        "nlg_stack_tensor": (i32, [vp, C.c_char_p, i32, C.POINTER(vp), C.POINTER(sz)]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(L, name)
        fn.restype, fn.argtypes = res, args
    _lib = L
    return L


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise NlgError(f"{what}: {lib().nlg_last_error().decode()}")


def init(device: int = -1) -> None:
    _check(lib().nlg_init(device), "nlg_init")


def device_name() -> str:
    b = C.create_string_buffer(256)
    _check(lib().nlg_device_name(b, 256), "nlg_device_name")
    return b.value.decode()


def device_info() -> tuple[int, str]:
    n = C.c_int(0)
    b = C.create_string_buffer(64)
    _check(lib().nlg_device_info(C.byref(n), b, 64), "nlg_device_info")
    return n.value, b.value.decode()


# ------------------------------------------------------------------ memory

class DeviceArray:
    """A device allocation of `nbytes`; element count in 4-byte slots is
    what kernels by name see (the reference's float count)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = lib().nlg_malloc(max(self.nbytes, 4))
        if not p:
            raise NlgError(f"nlg_malloc({nbytes}): {lib().nlg_last_error().decode()}")
        self.ptr = p

    @property
    def nfloats(self) -> int:
        return self.nbytes // 4

    def upload(self, arr: np.ndarray, offset: int = 0) -> "DeviceArray":
        a = np.ascontiguousarray(arr)
        if offset + a.nbytes > self.nbytes:
            raise NlgError("upload past the end of the buffer")
        _check(lib().nlg_upload(self.ptr + offset, a.ctypes.data, a.nbytes), "nlg_upload")
        return self

    def download(self, dtype=np.float32, count: Optional[int] = None, offset: int = 0) -> np.ndarray:
        dt = np.dtype(dtype)
        n = (self.nbytes - offset) // dt.itemsize if count is None else int(count)
        out = np.empty(n, dtype=dt)
        _check(lib().nlg_download(out.ctypes.data, self.ptr + offset, out.nbytes), "nlg_download")
        return out

    def zero(self, stream=None) -> None:
        _check(lib().nlg_zero(self.ptr, self.nbytes, stream), "nlg_zero")

    def free(self) -> None:
        if self.ptr:
            lib().nlg_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def as_buffer(self, nfloats: Optional[int] = None) -> Buffer:
        return Buffer(self.ptr, self.nfloats if nfloats is None else int(nfloats))


def to_device(arr: np.ndarray) -> DeviceArray:
    a = np.ascontiguousarray(arr)
    return DeviceArray(a.nbytes).upload(a)


def sync(stream=None) -> None:
    _check(lib().nlg_stream_sync(stream), "nlg_stream_sync")


# ------------------------------------------------------------------ kernels

def kernel_names() -> list[str]:
    L = lib()
    return [L.nlg_kernel_name(i).decode() for i in range(L.nlg_kernel_count())]


def kernel_abi(name: str) -> tuple[int, int]:
    nb, npu = C.c_uint32(0), C.c_uint32(0)
    _check(lib().nlg_kernel_abi(name.encode(), C.byref(nb), C.byref(npu)), "nlg_kernel_abi")
    return nb.value, npu.value


def dispatch(name: str, bufs: Sequence, push: Iterable[int], groups: int, stream=None,
             check: bool = True) -> int:
    """Run kernel `name` (reference ABI).  bufs: DeviceArray or (DeviceArray, nfloats)."""
    arr = (Buffer * max(len(bufs), 1))()
    for i, b in enumerate(bufs):
        if isinstance(b, tuple):
            arr[i] = b[0].as_buffer(b[1])
        else:
            arr[i] = b.as_buffer()
    pv = [int(p) & 0xFFFFFFFF for p in push]
    parr = (C.c_uint32 * max(len(pv), 1))(*pv)
    rc = lib().nlg_dispatch(name.encode(), arr, len(bufs), parr, len(pv), int(groups), stream)
    if check:
        _check(rc, f"dispatch {name}")
    return rc


def last_error() -> str:
    return lib().nlg_last_error().decode()


def pack_act_rows(x: DeviceArray, xq: DeviceArray, gamma: DeviceArray, seq: int, cols: int,
                  stream=None) -> None:
    _check(lib().nlg_pack_act_rows(x.ptr, xq.ptr, gamma.ptr, seq, cols, stream), "pack_act_rows")


def ternary_linear_i8(xq, gamma, w2, bias, beta, y, seq, out, cols, beta_per_row=False,
                      stream=None, rows_per_wave: int = 0, waves_per_block: int = 0) -> None:
    L = lib()
    bp = bias.ptr if bias is not None else None
    if rows_per_wave:
        rc = L.nlg_ternary_linear_i8_cfg(xq.ptr, gamma.ptr, w2.ptr, bp, beta.ptr, int(beta_per_row),
                                         y.ptr, seq, out, cols, rows_per_wave, waves_per_block or 4,
                                         stream)
    else:
        rc = L.nlg_ternary_linear_i8(xq.ptr, gamma.ptr, w2.ptr, bp, beta.ptr, int(beta_per_row),
                                     y.ptr, seq, out, cols, stream)
    _check(rc, "ternary_linear_i8")


def ternary_linear(x, w2, bias, beta, y, seq, out, cols, beta_per_row=False, gamma_out=None,
                   workspace=None, rows_per_wave: int = 0, stream=None) -> None:
    """pack-act-rows + ternary GEMV from f32 activations (one launch when fusable)."""
    L = lib()
    args = (x.ptr, w2.ptr, bias.ptr if bias is not None else None, beta.ptr, int(beta_per_row), y.ptr,
            gamma_out.ptr if gamma_out is not None else None, seq, out, cols)
    ws = workspace.ptr if workspace is not None else None
    wsb = workspace.nbytes if workspace is not None else 0
    if rows_per_wave:
        rc = L.nlg_ternary_linear_cfg(*args, rows_per_wave, ws, wsb, stream)
    else:
        rc = L.nlg_ternary_linear(*args, ws, wsb, stream)
    _check(rc, "ternary_linear")


def ternary_linear_noalloc(x, w2, bias, beta, y, seq, out, cols, beta_per_row=False, gamma_out=None,
                           stream=None) -> None:
    """ternary_linear with its scratch in the library's fixed array."""
    _check(lib().nlg_ternary_linear_noalloc(x.ptr, w2.ptr, _ptr(bias), beta.ptr, int(beta_per_row), y.ptr,
                                            _ptr(gamma_out), seq, out, cols, stream), "ternary_linear_noalloc")


def ternary_linear_workspace(seq: int, cols: int) -> int:
    return lib().nlg_ternary_linear_workspace(seq, cols)


def softmax_rows(a: DeviceArray, c: DeviceArray, rows: int, cols: int, stream=None) -> None:
    _check(lib().nlg_softmax_rows(a.ptr, c.ptr, rows, cols, stream), "softmax_rows")


def _ptr(a):
    return a.ptr if a is not None else None


def rms_ternary_linear(x, gain, eps, w2, bias, beta, y, seq, out, cols, beta_per_row=False,
                       stream=None) -> None:
    _check(lib().nlg_rms_ternary_linear(x.ptr, gain.ptr, eps, w2.ptr, _ptr(bias), beta.ptr,
                                        int(beta_per_row), y.ptr, seq, out, cols, stream),
           "rms_ternary_linear")


def ternary_linear_residual(x, w2, bias, beta, res, y, seq, out, cols, beta_per_row=False,
                            stream=None) -> None:
    _check(lib().nlg_ternary_linear_residual(x.ptr, w2.ptr, _ptr(bias), beta.ptr, int(beta_per_row),
                                             res.ptr, y.ptr, seq, out, cols, stream),
           "ternary_linear_residual")


def rms_ternary_swiglu(x, gain, eps, w2gu, beta, h, seq, dff, cols, beta_per_row=True,
                       stream=None) -> None:
    _check(lib().nlg_rms_ternary_swiglu(x.ptr, _ptr(gain), eps, w2gu.ptr, beta.ptr, int(beta_per_row),
                                        h.ptr, seq, dff, cols, stream), "rms_ternary_swiglu")


def rms_ternary_qkv_rope(x, gain, eps, w2, beta, q, kc, vc, co, si, pos, seq, heads, kvheads,
                         head_dim, max_seq, cols, beta_per_row=True, stream=None) -> None:
    _check(lib().nlg_rms_ternary_qkv_rope(x.ptr, gain.ptr, eps, w2.ptr, beta.ptr, int(beta_per_row),
                                          q.ptr, kc.ptr, vc.ptr, co.ptr, si.ptr, pos.ptr, seq, heads,
                                          kvheads, head_dim, max_seq, cols, stream),
           "rms_ternary_qkv_rope")


def rms_ternary_qkv_rope_prompt(x, gain, eps, w2, beta, q, kc, vc, co, si, pos, rows, qper, heads, kvheads,
                                head_dim, max_seq, cols, beta_per_row=True, stream=None) -> None:
    """Prompt rows: row r = sequence r // qper at position pos[0] + r % qper."""
    _check(lib().nlg_rms_ternary_qkv_rope_prompt(x.ptr, gain.ptr, eps, w2.ptr, beta.ptr, int(beta_per_row),
                                                 q.ptr, kc.ptr, vc.ptr, co.ptr, si.ptr, pos.ptr, rows, qper,
                                                 heads, kvheads, head_dim, max_seq, cols, stream),
           "rms_ternary_qkv_rope_prompt")


def rms_ternary_argmax(x, gain, eps, w2, beta, logits, argmax, seq, vocab, cols, workspace,
                       beta_per_row=False, stream=None) -> None:
    _check(lib().nlg_rms_ternary_argmax(x.ptr, gain.ptr, eps, w2.ptr, beta.ptr, int(beta_per_row),
                                        logits.ptr, argmax.ptr, seq, vocab, cols, workspace.ptr,
                                        workspace.nbytes, stream), "rms_ternary_argmax")


def rms_ternary_argmax_workspace(seq: int, vocab: int) -> int:
    return lib().nlg_rms_ternary_argmax_workspace(seq, vocab)


def decode_attn_f16(q, kc, vc, pos, out, batch, heads, kvheads, head_dim, max_seq, workspace,
                    stream=None) -> None:
    _check(lib().nlg_decode_attn_f16(q.ptr, kc.ptr, vc.ptr, pos.ptr, out.ptr, batch, heads, kvheads,
                                     head_dim, max_seq, workspace.ptr, workspace.nbytes, stream),
           "decode_attn_f16")


def decode_attn_f16_chunks(q, kc, vc, pos, batch, heads, kvheads, head_dim, max_seq, workspace,
                           stream=None) -> None:
    _check(lib().nlg_decode_attn_f16_chunks(q.ptr, kc.ptr, vc.ptr, pos.ptr, batch, heads, kvheads,
                                            head_dim, max_seq, workspace.ptr, workspace.nbytes, stream),
           "decode_attn_f16_chunks")


def prefill_attn_f16(q, kc, vc, pos, rows, qper, heads, kvheads, head_dim, max_seq, ctx,
                     stream=None) -> None:
    """Causal attention of rows prompt rows (row r = sequence r // qper at
    position pos[0] + r % qper) over fp16 caches; ctx [rows][heads*head_dim]."""
    _check(lib().nlg_prefill_attn_f16(q.ptr, kc.ptr, vc.ptr, pos.ptr, rows, qper, heads, kvheads, head_dim,
                                      max_seq, ctx.ptr, stream), "prefill_attn_f16")


def prefill_attn_ternary_linear_residual(q, kc, vc, pos, rows, qper, heads, kvheads, head_dim, max_seq, ctx_ws,
                                         w2, bias, beta, res, y, out, beta_per_row=False, stream=None) -> None:
    """That attention, then y = res + linear(ctx) (the stack's prefill form)."""
    _check(lib().nlg_prefill_attn_ternary_linear_residual(
        q.ptr, kc.ptr, vc.ptr, pos.ptr, rows, qper, heads, kvheads, head_dim, max_seq, ctx_ws.ptr, w2.ptr,
        _ptr(bias), beta.ptr, int(beta_per_row), res.ptr, y.ptr, out, stream),
        "prefill_attn_ternary_linear_residual")


def decode_attn_paged_f16_workspace(batch, heads, kvheads, head_dim, bs, mbps) -> int:
    return int(lib().nlg_decode_attn_paged_f16_workspace(batch, heads, kvheads, head_dim, bs, mbps))


def decode_attn_paged_f16(q, kpool, vpool, lens, table, npool, out, batch, heads, kvheads, head_dim, bs, mbps,
                          workspace, stream=None) -> None:
    _check(lib().nlg_decode_attn_paged_f16(q.ptr, kpool.ptr, vpool.ptr, lens.ptr, table.ptr, npool, out.ptr, batch,
                                           heads, kvheads, head_dim, bs, mbps, workspace.ptr, workspace.nbytes,
                                           stream), "decode_attn_paged_f16")


def cache_append_paged_f16(src, lens, table, npool, pool, batch, kvdim, bs, mbps, stream=None) -> None:
    _check(lib().nlg_cache_append_paged_f16(src.ptr, lens.ptr, table.ptr, npool, pool.ptr, batch, kvdim, bs, mbps,
                                            stream), "cache_append_paged_f16")


def decode_attn_stream_f16_workspace(batch, heads, kvheads, head_dim, nsink, win) -> int:
    return int(lib().nlg_decode_attn_stream_f16_workspace(batch, heads, kvheads, head_dim, nsink, win))


def decode_attn_stream_f16(q, kc, vc, pos, co, si, out, batch, heads, kvheads, head_dim, nsink, win, workspace,
                           stream=None) -> None:
    """StreamingLLM decode attention over fp16 ring caches [batch][kvheads][nsink+win][head_dim]."""
    _check(lib().nlg_decode_attn_stream_f16(q.ptr, kc.ptr, vc.ptr, pos.ptr, co.ptr, si.ptr, out.ptr, batch, heads,
                                            kvheads, head_dim, nsink, win, workspace.ptr, workspace.nbytes, stream),
           "decode_attn_stream_f16")


def attn_entries_f16_workspace(batch, heads, kvheads, head_dim, ne) -> int:
    return int(lib().nlg_attn_entries_f16_workspace(batch, heads, kvheads, head_dim, ne))


def attn_entries_f16(q, kc, vc, ent, qrank, co, si, out, batch, heads, kvheads, head_dim, nslots, ne, trows,
                     workspace, stream=None) -> None:
    """attn-stream-entries over fp16 caches [batch][kvheads][nslots][head_dim]; ent [batch][ne][2] int32."""
    _check(lib().nlg_attn_entries_f16(q.ptr, kc.ptr, vc.ptr, ent.ptr, qrank.ptr, co.ptr, si.ptr, out.ptr, batch,
                                      heads, kvheads, head_dim, nslots, ne, trows, workspace.ptr, workspace.nbytes,
                                      stream), "attn_entries_f16")


def block_copy_f16(kpool, vpool, pairs, n, npool, bs, kvdim, stream=None) -> None:
    _check(lib().nlg_block_copy_f16(kpool.ptr, vpool.ptr, pairs.ptr, n, npool, bs, kvdim, stream), "block_copy_f16")


def cache_append_ring_f16(src, pos, cache, batch, kvheads, head_dim, nsink, win, stream=None) -> None:
    _check(lib().nlg_cache_append_ring_f16(src.ptr, pos.ptr, cache.ptr, batch, kvheads, head_dim, nsink, win,
                                           stream), "cache_append_ring_f16")


def repack_i8_to_2bit(wp, out, cols, w2, nbad=None, stream=None) -> None:
    """int8-lane ternary words [out x ceil(cols/4)] -> 2-bit words [out x ceil(cols/16)]."""
    _check(lib().nlg_repack_i8_to_2bit(wp.ptr, out, cols, w2.ptr, _ptr(nbad), stream), "repack_i8_to_2bit")


def repack_packed_to_2bit(wpk, out, cols, pk, fcount, w2, nbad=None, stream=None) -> None:
    """base-4 codes in f32 [out x fcount] -> 2-bit words [out x ceil(cols/16)]."""
    _check(lib().nlg_repack_packed_to_2bit(wpk.ptr, out, cols, pk, fcount, w2.ptr, _ptr(nbad), stream),
           "repack_packed_to_2bit")


def ternary_tiled_register(w2, rows, cols, stream=None) -> None:
    """Keep a copy of 2-bit weights [rows x cols/16] in the prompt GEMM's load order."""
    _check(lib().nlg_ternary_tiled_register(w2.ptr, rows, cols, stream), "ternary_tiled_register")


def ternary_tiled_unregister(w2) -> None:
    """Drop the tiled copy of w2 (a no-op when there is none)."""
    _check(lib().nlg_ternary_tiled_unregister(w2.ptr), "ternary_tiled_unregister")


def attn_ternary_linear_residual(workspace, batch, heads, kvheads, head_dim, max_seq, w2, bias, beta,
                                 res, y, out, beta_per_row=False, stream=None) -> None:
    _check(lib().nlg_attn_ternary_linear_residual(workspace.ptr, workspace.nbytes, batch, heads, kvheads,
                                                  head_dim, max_seq, w2.ptr, _ptr(bias), beta.ptr,
                                                  int(beta_per_row), res.ptr, y.ptr, out, stream),
           "attn_ternary_linear_residual")


def decode_attn_f16_workspace(batch, heads, kvheads, head_dim, max_seq) -> int:
    return lib().nlg_decode_attn_f16_workspace(batch, heads, kvheads, head_dim, max_seq)


def fill_normal(dev, n: int, seed: int, sigma: float = 1.0, causal: int = 0, stream=None) -> None:
    _check(lib().nlg_fill_normal(dev.ptr, n, seed, sigma, causal, stream), "fill_normal")


class Stack:
    """The random-initialised ternary decoder stack (nlg_stack_* in nlgpu.h)."""

    def __init__(self, layers, d_model, heads, kv_heads, head_dim, d_ff, vocab, max_seq, batch,
                 rms_eps=1e-5, rope_theta=500000.0, seed=20260921 + 5):
        self.cfg = StackConfig(layers, d_model, heads, kv_heads, head_dim, d_ff, vocab, max_seq,
                               batch, rms_eps, rope_theta, seed)
        h = C.c_void_p()
        _check(lib().nlg_stack_create(C.byref(self.cfg), C.byref(h)), "stack_create")
        self.h = h.value

    def start(self, prompts: np.ndarray) -> None:
        p = np.ascontiguousarray(prompts, np.int32)
        assert p.ndim == 2 and p.shape[0] == self.cfg.batch
        _check(lib().nlg_stack_start(self.h, p.ctypes.data, p.shape[1]), "stack_start")

    def prefill(self, prompts: np.ndarray) -> None:
        p = np.ascontiguousarray(prompts, np.int32)
        assert p.ndim == 2 and p.shape[0] == self.cfg.batch
        _check(lib().nlg_stack_prefill(self.h, p.ctypes.data, p.shape[1]), "stack_prefill")

    def prefill_trace(self, prompts: np.ndarray) -> np.ndarray:
        """prefill(prompts), returning the prompt rows' residual stream
        [layers + 1, batch * n_prompt, d_model]: the embedded rows, then the
        rows after each layer."""
        p = np.ascontiguousarray(prompts, np.int32)
        assert p.ndim == 2 and p.shape[0] == self.cfg.batch
        c = self.cfg
        xs = np.empty((c.layers + 1) * p.size * c.d_model, np.float32)
        _check(lib().nlg_stack_prefill_trace(self.h, p.ctypes.data, p.shape[1], xs.ctypes.data),
               "stack_prefill_trace")
        return xs.reshape(c.layers + 1, p.size, c.d_model)

    def step(self, steps: int = 1, graph: bool = True) -> None:
        _check(lib().nlg_stack_step(self.h, steps, int(graph)), "stack_step")

    def step_trace(self) -> np.ndarray:
        """One eager step; returns the residual stream [layers + 1, batch,
        d_model]: the embedded token, then the stream after each layer."""
        c = self.cfg
        xs = np.empty((c.layers + 1) * c.batch * c.d_model, np.float32)
        _check(lib().nlg_stack_step_trace(self.h, xs.ctypes.data), "stack_step_trace")
        return xs.reshape(c.layers + 1, c.batch, c.d_model)

    def position(self) -> int:
        p = C.c_uint32(0)
        _check(lib().nlg_stack_position(self.h, C.byref(p)), "stack_position")
        return p.value

    def tokens(self):
        n = self.cfg.batch * self.cfg.max_seq
        t, g = np.empty(n, np.int32), np.empty(n, np.int32)
        _check(lib().nlg_stack_tokens(self.h, t.ctypes.data, g.ctypes.data), "stack_tokens")
        return t.reshape(self.cfg.batch, -1), g.reshape(self.cfg.batch, -1)

    def logits(self) -> np.ndarray:
        out = np.empty(self.cfg.batch * self.cfg.vocab, np.float32)
        _check(lib().nlg_stack_logits(self.h, out.ctypes.data), "stack_logits")
        return out.reshape(self.cfg.batch, -1)

    def tensor(self, name: str, layer: int = -1, dtype=np.float32) -> np.ndarray:
        p, n = C.c_void_p(), C.c_size_t(0)
        _check(lib().nlg_stack_tensor(self.h, name.encode(), layer, C.byref(p), C.byref(n)),
               f"stack_tensor {name}")
        dt = np.dtype(dtype)
        out = np.empty(n.value // dt.itemsize, dt)
        _check(lib().nlg_download(out.ctypes.data, p.value, out.nbytes), "download")
        return out

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().nlg_stack_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ------------------------------------------------------------- events, graphs

class Event:
    def __init__(self):
        self.ev = lib().nlg_event_create()
        if not self.ev:
            raise NlgError(last_error())

    def record(self, stream=None) -> None:
        _check(lib().nlg_event_record(self.ev, stream), "event_record")

    def elapsed_ms(self, later: "Event") -> float:
        ms = C.c_float(0)
        _check(lib().nlg_event_elapsed_ms(self.ev, later.ev, C.byref(ms)), "event_elapsed")
        return ms.value

    def __del__(self):
        try:
            lib().nlg_event_destroy(self.ev)
        except Exception:
            pass


def graph_begin(stream=None) -> None:
    _check(lib().nlg_graph_begin(stream), "graph_begin")


def graph_end(stream=None):
    g = C.c_void_p()
    _check(lib().nlg_graph_end(stream, C.byref(g)), "graph_end")
    return g.value


def graph_launch(g, stream=None) -> None:
    _check(lib().nlg_graph_launch(g, stream), "graph_launch")


def graph_destroy(g) -> None:
    lib().nlg_graph_destroy(g)


# ------------------------------------------------------------- data formats

def pack_ternary(trits: np.ndarray) -> np.ndarray:
    """Pack an [out, cols] array of {-1,0,+1} (or -2) into the reference's
    2-bit words: 16 fields per u32, field f in bits 2f..2f+1, codes
    +1 -> 01, -1 -> 11, 0 -> 00, -2 -> 10 (test/ternary-kernel-test.el:40-50).
    Returns uint32 [out, ceil(cols/16)]."""
    t = np.asarray(trits)
    out, cols = t.shape
    wng = (cols + 15) // 16
    codes = np.zeros((out, wng * 16), dtype=np.uint32)
    codes[:, :cols] = (t.astype(np.int64) & 3).astype(np.uint32)
    codes = codes.reshape(out, wng, 16)
    shifts = (2 * np.arange(16, dtype=np.uint32))
    return np.bitwise_or.reduce(codes << shifts, axis=2).astype(np.uint32)


def unpack_ternary(words: np.ndarray, cols: int) -> np.ndarray:
    """Inverse of pack_ternary, decoding by sign extension as ternary-rows
    does (lisp/nelisp-gpu-kernels.el:728-743): 00 0, 01 +1, 11 -1, 10 -2."""
    w = np.asarray(words, dtype=np.uint32)
    out, wng = w.shape
    f = np.arange(16, dtype=np.uint32)
    codes = (w[:, :, None] >> (2 * f)) & 3
    vals = np.where(codes >= 2, codes.astype(np.int64) - 4, codes.astype(np.int64)).astype(np.int8)
    return vals.reshape(out, wng * 16)[:, :cols]


_M64 = (1 << 64) - 1


def splitmix64(seed: int, n: int) -> np.ndarray:
    """n outputs of SplitMix64 with state seed + (i+1)*golden (counter-based,
    so any slice is reproducible independently)."""
    with np.errstate(over="ignore"):
        i = np.arange(1, n + 1, dtype=np.uint64)
        z = np.uint64(seed & _M64) + i * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, n: int) -> np.ndarray:
    """float64 in [0, 1) from the top 53 bits."""
    return (splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))


def normal(seed: int, n: int, sigma: float = 1.0) -> np.ndarray:
    """float32 N(0, sigma^2) by Box-Muller in double."""
    m = (n + 1) // 2
    u = uniform(seed, 2 * m)
    u1 = 1.0 - u[:m]  # (0, 1]
    u2 = u[m:]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.concatenate([r * np.cos(2 * np.pi * u2), r * np.sin(2 * np.pi * u2)])[:n]
    return (sigma * z).astype(np.float32)


def trits(seed: int, shape) -> np.ndarray:
    """{-1, 0, +1} with probabilities {0.25, 0.5, 0.25}."""
    n = int(np.prod(shape))
    u = uniform(seed, n)
    t = np.where(u < 0.25, -1, np.where(u < 0.75, 0, 1)).astype(np.int8)
    return t.reshape(shape)


def normal_pairs(seed: int, n: int) -> np.ndarray:
    """float32 N(0,1) as the device generator draws it: elements 2p and 2p+1
    share u1 = 1 - u(2p), u2 = u(2p+1) and take r cos(2 pi u2), r sin(2 pi u2)."""
    m = (n + 1) // 2
    u = uniform(seed, 2 * m)
    r = np.sqrt(-2.0 * np.log(1.0 - u[0::2]))
    t = 6.283185307179586 * u[1::2]
    z = np.empty(2 * m)
    z[0::2], z[1::2] = r * np.cos(t), r * np.sin(t)
    return z[:n].astype(np.float32)


def stack_tensor_seed(seed: int, layer: int, tensor: int) -> int:
    """Seed of one tensor of the decoder stack: per layer, tensors 0..8 are
    q, k, v, o, gate, up, down, attention gain, FFN gain; after the last
    layer, 0..2 are the LM head, the final gain and the embedding."""
    return (seed + 1000003 * (layer + 1) + tensor) & _M64
