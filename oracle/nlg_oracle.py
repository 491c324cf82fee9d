"""ctypes binding of the CPU restatement (libnlg_oracle.so).

TEST INFRASTRUCTURE ONLY: the checker the MI355X kernels are compared with,
and the CPU baseline bench.py times.  Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg import this module; the product library and
hosts never load it.  See nlg_oracle.c for the per-kernel citations of
lisp/nelisp-gpu-kernels.el.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libnlg_oracle.so")

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = C.CDLL(LIB_PATH)
        vp, u32, i32 = C.c_void_p, C.c_uint32, C.c_int
        L.or_dispatch.restype = i32
        L.or_dispatch.argtypes = [C.c_char_p, C.POINTER(C.c_void_p), C.POINTER(u32), u32,
                                  C.POINTER(u32), u32, u32]
        L.or_kernel_count.restype = i32
        L.or_kernel_name.restype = C.c_char_p
        L.or_kernel_name.argtypes = [i32]
        L.or_kernel_abi.restype = i32
        L.or_kernel_abi.argtypes = [C.c_char_p, C.POINTER(u32), C.POINTER(u32)]
        L.or_ternary_linear_i8.restype = None
        L.or_ternary_linear_i8.argtypes = [vp, vp, vp, vp, vp, i32, vp, u32, u32, u32]
        L.or_ternary_acc_i8.restype = None
        L.or_ternary_acc_i8.argtypes = [vp, vp, vp, u32, u32, u32]
        L.or_pack_act_rows.restype = None
        L.or_pack_act_rows.argtypes = [vp, vp, vp, u32, u32]
        L.or_softmax_rows.restype = None
        L.or_softmax_rows.argtypes = [vp, vp, u32, u32]
        L.or_rmsnorm_rows.restype = None
        L.or_rmsnorm_rows.argtypes = [vp, vp, C.c_float, vp, u32, u32]
        L.or_decode_attn_f16.restype = None
        L.or_decode_attn_f16.argtypes = [vp, vp, vp, u32, vp, u32, u32, u32, u32, u32]
        L.or_decode_attn_paged_f16.restype = None
        L.or_decode_attn_paged_f16.argtypes = [vp, vp, vp, vp, vp, u32, vp, u32, u32, u32, u32, u32, u32]
        L.or_decode_attn_stream_f16.restype = None
        L.or_decode_attn_stream_f16.argtypes = [vp, vp, vp, vp, vp, vp, vp, u32, u32, u32, u32, u32, u32]
        L.or_attn_entries_f16.restype = None
        L.or_attn_entries_f16.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, u32]
        L.or_repack_i8_2bit.restype = u32
        L.or_repack_i8_2bit.argtypes = [vp, u32, u32, vp]
        L.or_repack_packed_2bit.restype = u32
        L.or_repack_packed_2bit.argtypes = [vp, u32, u32, u32, u32, vp]
        L.or_threads.restype = i32
        L.or_set_threads.argtypes = [i32]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data if a is not None else None


def kernel_names() -> list[str]:
    L = lib()
    return [L.or_kernel_name(i).decode() for i in range(L.or_kernel_count())]


def kernel_abi(name: str) -> tuple[int, int]:
    nb, npu = C.c_uint32(0), C.c_uint32(0)
    if lib().or_kernel_abi(name.encode(), C.byref(nb), C.byref(npu)):
        raise KeyError(name)
    return nb.value, npu.value


def dispatch(name: str, bufs: Sequence[np.ndarray], push: Sequence[int], groups: int) -> None:
    """Run kernel `name` over numpy buffers in place.  Each buffer must be a
    C-contiguous 4-byte-element array (float32 or uint32 views); the same
    array may appear twice (in-place kernels)."""
    n = len(bufs)
    ptrs = (C.c_void_p * max(n, 1))()
    sizes = (C.c_uint32 * max(n, 1))()
    for i, b in enumerate(bufs):
        assert b.flags["C_CONTIGUOUS"] and b.dtype.itemsize == 4, (name, i)
        ptrs[i] = b.ctypes.data
        sizes[i] = b.size
    pv = [int(p) & 0xFFFFFFFF for p in push]
    parr = (C.c_uint32 * max(len(pv), 1))(*pv)
    if lib().or_dispatch(name.encode(), ptrs, sizes, n, parr, len(pv), int(groups)):
        raise ValueError(f"oracle: bad dispatch {name}")


def pack_act_rows(x: np.ndarray, seq: int, cols: int):
    x = np.ascontiguousarray(x, dtype=np.float32)
    ng = (cols + 3) // 4
    xq = np.zeros(seq * ng, dtype=np.uint32)
    gamma = np.zeros(seq, dtype=np.float32)
    lib().or_pack_act_rows(_p(x), _p(xq), _p(gamma), seq, cols)
    return xq, gamma


def ternary_acc_i8(xq: np.ndarray, w2: np.ndarray, seq: int, out: int, cols: int) -> np.ndarray:
    acc = np.zeros(seq * out, dtype=np.int32)
    lib().or_ternary_acc_i8(_p(np.ascontiguousarray(xq, np.uint32)),
                            _p(np.ascontiguousarray(w2, np.uint32)), _p(acc), seq, out, cols)
    return acc


def ternary_linear_i8(xq, gamma, w2, bias, beta, seq, out, cols, beta_per_row=False) -> np.ndarray:
    y = np.zeros(seq * out, dtype=np.float32)
    b = np.ascontiguousarray(bias, np.float32) if bias is not None else None
    lib().or_ternary_linear_i8(_p(np.ascontiguousarray(xq, np.uint32)),
                               _p(np.ascontiguousarray(gamma, np.float32)),
                               _p(np.ascontiguousarray(w2, np.uint32)), _p(b),
                               _p(np.ascontiguousarray(beta, np.float32)), int(beta_per_row),
                               _p(y), seq, out, cols)
    return y


def softmax_rows(a: np.ndarray, rows: int, cols: int) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    c = np.empty_like(a)
    lib().or_softmax_rows(_p(a), _p(c), rows, cols)
    return c


def rmsnorm_rows(x: np.ndarray, gain: np.ndarray, eps: float, rows: int, cols: int) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows * cols, np.float32)
    lib().or_rmsnorm_rows(_p(x), _p(np.ascontiguousarray(gain, np.float32)), float(eps), _p(y), rows, cols)
    return y


def decode_attn_f16(q, kc, vc, pos, B, heads, kvheads, hd, max_seq) -> np.ndarray:
    """kc, vc: uint16 fp16 bit patterns [B][kvheads][max_seq][hd]."""
    out = np.empty(B * heads * hd, np.float32)
    lib().or_decode_attn_f16(_p(np.ascontiguousarray(q, np.float32)),
                             _p(np.ascontiguousarray(kc, np.uint16)),
                             _p(np.ascontiguousarray(vc, np.uint16)), int(pos), _p(out), B, heads,
                             kvheads, hd, max_seq)
    return out


def decode_attn_paged_f16(q, kp, vp, lens, table, npool, B, heads, kvheads, hd, bs, mbps) -> np.ndarray:
    """kp, vp: uint16 fp16 pools [block][bs][kvheads][hd]; lens int32 [B]; table int32 [B x mbps]."""
    out = np.empty(B * heads * hd, np.float32)
    lib().or_decode_attn_paged_f16(_p(np.ascontiguousarray(q, np.float32)), _p(np.ascontiguousarray(kp, np.uint16)),
                                   _p(np.ascontiguousarray(vp, np.uint16)), _p(np.ascontiguousarray(lens, np.int32)),
                                   _p(np.ascontiguousarray(table, np.int32)), npool, _p(out), B, heads, kvheads, hd,
                                   bs, mbps)
    return out


def decode_attn_stream_f16(q, kc, vc, pos, co, si, B, heads, kvheads, hd, nsink, win) -> np.ndarray:
    """kc, vc: uint16 fp16 ring caches [B][kvheads][nsink+win][hd]; pos int32 [B]; co, si f32 [>= cap][hd/2]."""
    out = np.empty(B * heads * hd, np.float32)
    lib().or_decode_attn_stream_f16(_p(np.ascontiguousarray(q, np.float32)), _p(np.ascontiguousarray(kc, np.uint16)),
                                    _p(np.ascontiguousarray(vc, np.uint16)), _p(np.ascontiguousarray(pos, np.int32)),
                                    _p(np.ascontiguousarray(co, np.float32)), _p(np.ascontiguousarray(si, np.float32)),
                                    _p(out), B, heads, kvheads, hd, nsink, win)
    return out


def attn_entries_f16(q, kc, vc, ent, qrank, co, si, B, heads, kvheads, hd, nslots, ne, trows) -> np.ndarray:
    """kc, vc: uint16 fp16 caches [B][kvheads][nslots][hd]; ent int32 [B][ne][2] (slot, rank); qrank int32 [B];
    co, si f32 [trows][hd/2]."""
    out = np.empty(B * heads * hd, np.float32)
    lib().or_attn_entries_f16(_p(np.ascontiguousarray(q, np.float32)), _p(np.ascontiguousarray(kc, np.uint16)),
                              _p(np.ascontiguousarray(vc, np.uint16)), _p(np.ascontiguousarray(ent, np.int32)),
                              _p(np.ascontiguousarray(qrank, np.int32)), _p(np.ascontiguousarray(co, np.float32)),
                              _p(np.ascontiguousarray(si, np.float32)), _p(out), B, heads, kvheads, hd, nslots, ne,
                              trows)
    return out


def block_copy_f16(kpool, vpool, pairs, npool, bs, kvdim) -> None:
    """block-copy (kernels.el:1184-1193) on both fp16 pools [npool][bs*kvdim], in place, pairs (src, dst) in
    order; pairs naming a block outside [0, npool) are skipped."""
    kp, vp = kpool.reshape(npool, bs * kvdim), vpool.reshape(npool, bs * kvdim)
    for src, dst in np.asarray(pairs, np.int64).reshape(-1, 2):
        if 0 <= src < npool and 0 <= dst < npool:
            kp[dst] = kp[src]
            vp[dst] = vp[src]


def cache_append_ring_f16(cache, src, pos, B, kvheads, hd, nsink, win) -> None:
    """cache-append-ring (kernels.el:396-403) into fp16 ring caches [B][kvheads][nsink+win][hd], in place:
    row s of src [B x kvheads*hd] (rounded to fp16, nearest even) at the slot of pos[s]; negative pos skipped."""
    cap = nsink + win
    c = cache.reshape(B, kvheads, cap, hd)
    for s in range(B):
        p = int(pos[s])
        if p < 0:
            continue
        slot = p if p < nsink else nsink + (p - nsink) % win
        c[s, :, slot, :] = np.asarray(src, np.float32).reshape(B, kvheads, hd)[s].astype(np.float16).view(np.uint16)


def repack_i8_2bit(wp, out, cols):
    """int8-lane words [out x ceil(cols/4)] -> (2-bit words [out x ceil(cols/16)], count unrepresentable)."""
    w2 = np.empty((out, (cols + 15) // 16), np.uint32)
    bad = lib().or_repack_i8_2bit(_p(np.ascontiguousarray(wp, np.uint32)), out, cols, _p(w2))
    return w2, int(bad)


def repack_packed_2bit(wpk, out, cols, pk, fcount):
    """base-4 codes in f32 [out x fcount] -> (2-bit words, count of code 3)."""
    w2 = np.empty((out, (cols + 15) // 16), np.uint32)
    bad = lib().or_repack_packed_2bit(_p(np.ascontiguousarray(wpk, np.float32)), out, cols, pk, fcount, _p(w2))
    return w2, int(bad)


def threads() -> int:
    return lib().or_threads()


def set_threads(n: int) -> None:
    lib().or_set_threads(n)
