"""numpy/ctypes front end of the CPU checker libraries.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package.

  Oracle()     -> oracle/liboracle.so, the C restatement (fl_oracle.c)
  Oracle(ref=True) -> oracle/_ref/libflref.so, the reference's own code
                  compiled from /root/reference (exists only where that tree
                  does; used to write tests/golden fixtures)
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libflref.so")

F32, Q8_0, Q5_0, Q4_K, Q6_K, IQ2_XXS, IQ3_XXS = 0, 1, 2, 3, 4, 5, 6
BLK = {F32: (1, 4), Q8_0: (32, 34), Q5_0: (32, 22), Q4_K: (256, 144), Q6_K: (256, 210),
       IQ2_XXS: (256, 66), IQ3_XXS: (256, 98)}


def row_bytes(fmt, cols):
    e, b = BLK[fmt]
    return (cols // e) * b


def xq_offset(cols):
    return (cols * 4 + 15) & ~15


def xqk_offset(cols):
    return xq_offset(cols) + (((cols // 32) * 36 + 15) & ~15)


def x_alloc_bytes(cols):
    return xqk_offset(cols) + (cols // 256) * 292


def col_stride_floats(cols):
    """Per-column stride used by tests: 128-B padded (src/model/decoder.cpp:412-416)."""
    return ((x_alloc_bytes(cols) + 127) & ~127) // 4


_P, _U32, _U64, _F, _I = C.c_void_p, C.c_uint32, C.c_uint64, C.c_float, C.c_int


def _ptr(a):
    return None if a is None else a.ctypes.data


class Oracle:
    def __init__(self, ref: bool = False):
        path = REF_SO if ref else ORACLE_SO
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built (make -C oracle{' ref' if ref else ''})")
        self.ref = ref
        L = C.CDLL(path)
        pre = "ref_" if ref else "orc_"
        self._half2float = getattr(L, pre + "half2float")
        self._half2float.restype, self._half2float.argtypes = _F, [C.c_uint16]
        self._float2half = getattr(L, pre + "float2half")
        self._float2half.restype, self._float2half.argtypes = C.c_uint16, [_F]
        self._dequant = getattr(L, pre + "dequant_rows")
        self._dequant.restype, self._dequant.argtypes = None, [_I, _P, _U32, _U32, _P]
        self._act = getattr(L, pre + "act_q8")
        self._act.restype, self._act.argtypes = None, [_P, _U32]
        if ref:
            self._sd = L.ref_stream_dot
            self._sd.restype = None
            self._sd.argtypes = [_I, _P, _U32, _U32, _P, _P, _U32, _U32, _U32, _I, _U32, _U32,
                                 _P, _U64]
            self._sdmt = L.ref_stream_dot_mt
            self._sdmt.restype = None
            self._sdmt.argtypes = [_I, _P, _U32, _U32, _P, _P, _U32, _U32, _U32, _I, _U32, _U32, _I]
            self._canon = L.ref_stream_dot_canonical
            self._canon.restype = None
            self._canon.argtypes = [_I, _P, _U32, _U32, _P, _P, _U32, _U32, _U32]
        else:
            self._sd = L.orc_stream_dot
            self._sd.restype = None
            self._sd.argtypes = [_I, _P, _U32, _U32, _P, _P, _U32, _U32, _U32, _I, _U32, _U32]
            self._sdmt = L.orc_stream_dot_mt
            self._sdmt.restype = None
            self._sdmt.argtypes = [_I, _P, _U32, _U32, _P, _P, _U32, _U32, _U32, _I, _U32, _U32, _I]
            for n, args, res in [
                ("orc_dot_i8_q8_0", [_P, _P, _U32], _F), ("orc_dot_i8_q5_0", [_P, _P, _U32], _F),
                ("orc_dot_i8_iq", [_I, _P, _P, _U32], _F), ("orc_iq2_grid", [_I], C.c_uint64),
                ("orc_iq3_grid", [_I], _U32), ("orc_iq_signs", [_U32], C.c_uint8),
                ("orc_dot_i8k_q4_K", [_P, _P, _U32], _F),
                ("orc_dot_i8k_q6_K", [_P, _P, _U32], _F), ("orc_dot_i8_q4_K", [_P, _P, _U32], _F),
                ("orc_dot_i8_q6_K", [_P, _P, _U32], _F), ("orc_dot_row", [_I, _P, _P, _U32], _F),
                ("orc_q4k_scale_min", [_I, _P, _P, _P], None),
                ("orc_quantize_q8_1_block", [_P, _P], None),
                ("orc_quantize_q8_K_block", [_P, _P], None)]:
                f = getattr(L, n)
                f.restype, f.argtypes = res, args
                setattr(self, n[4:], f)
        self._rmsnorm = getattr(L, pre + "rmsnorm")
        self._rmsnorm.restype = None
        self._rmsnorm.argtypes = [_P, _P, _P, _F, _U32]
        for n in ("router_sel", "silu_mul", "wmerge"):
            setattr(self, "_" + n, getattr(L, pre + n))
        self._router_sel.restype = None
        self._router_sel.argtypes = [_P, _U32, _U32, _U32, _F, _P, _P]
        self._silu_mul.restype = None
        self._silu_mul.argtypes = [_P, _P, _P, _U32]
        self._wmerge.restype = None
        self._wmerge.argtypes = [_P, _P, _P, _P, _P, _F, _U32, _U32, _U32]
        self.lib = L

    # ---- scalar conversions
    def half2float(self, h: int) -> float:
        return self._half2float(h)

    def float2half(self, f: float) -> int:
        return self._float2half(f)

    # ---- dequant / act quant
    def dequant(self, fmt, w: np.ndarray, rows, cols) -> np.ndarray:
        w = np.ascontiguousarray(w, dtype=np.uint8)
        assert w.size >= rows * row_bytes(fmt, cols)
        out = np.empty(rows * cols, dtype=np.float32)
        self._dequant(fmt, _ptr(w), rows, cols, _ptr(out))
        return out.reshape(rows, cols)

    def act_q8(self, x: np.ndarray, cols: int | None = None) -> np.ndarray:
        """One column: returns the full fl_x_alloc_bytes(cols) buffer (uint8)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        cols = x.size if cols is None else cols
        buf = np.zeros(x_alloc_bytes(cols) + 64, dtype=np.uint8)
        off = (-buf.ctypes.data) % 16
        view = buf[off:off + x_alloc_bytes(cols)]
        view[:cols * 4] = x[:cols].view(np.uint8)
        self._act(view.ctypes.data, cols)
        return view.copy()

    def act_q8_cols(self, xs: np.ndarray, stride_floats: int | None = None) -> np.ndarray:
        """[nx, cols] -> float32 buffer of nx columns at stride_floats, appendices filled."""
        nx, cols = xs.shape
        st = col_stride_floats(cols) if stride_floats is None else stride_floats
        buf = np.zeros(nx * st + 16, dtype=np.float32)
        off = ((-buf.ctypes.data) % 16) // 4
        view = buf[off:off + nx * st]
        for p in range(nx):
            col = view[p * st:(p + 1) * st]
            col[:cols] = xs[p]
            self._act(col.ctypes.data, cols)
        return view.copy()

    # ---- dots
    def stream_dot(self, fmt, w, rows, cols, xbuf, y, nx=1, xstride=0, ystride=0, fast=True,
                   i8_mask=0b11110, i8k_mask=0b11000, threads=1, id_slot=None, estride=0):
        """y += W x (exec_task_cpu); xbuf is the float32 column buffer (appendices set)."""
        w = np.ascontiguousarray(w, dtype=np.uint8)
        xbuf = np.ascontiguousarray(xbuf, dtype=np.float32)
        assert y.dtype == np.float32 and y.flags.c_contiguous
        if self.ref and threads > 1 and id_slot is None:
            self._sdmt(fmt, _ptr(w), rows, cols, _ptr(xbuf), _ptr(y), nx, xstride, ystride,
                       int(fast), i8_mask, i8k_mask, threads)
            return y
        if self.ref:
            slot = None if id_slot is None else np.array([id_slot], dtype=np.uint32)
            self._sd(fmt, _ptr(w), rows, cols, _ptr(xbuf), _ptr(y), nx, xstride, ystride,
                     int(fast), i8_mask, i8k_mask, _ptr(slot), estride)
            return y
        wb = w
        if id_slot is not None:
            wb = w[id_slot * estride:]
        if threads > 1:
            self._sdmt(fmt, _ptr(wb), rows, cols, _ptr(xbuf), _ptr(y), nx, xstride, ystride,
                       int(fast), i8_mask, i8k_mask, threads)
        else:
            self._sd(fmt, _ptr(wb), rows, cols, _ptr(xbuf), _ptr(y), nx, xstride, ystride,
                     int(fast), i8_mask, i8k_mask)
        return y

    # ---- MoE glue
    def router_sel(self, logits, top_k, norm=1, scale=1.0):
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        ids = np.zeros(top_k, dtype=np.uint32)
        gates = np.zeros(top_k, dtype=np.float32)
        self._router_sel(_ptr(logits), logits.size, top_k, norm, scale, _ptr(ids), _ptr(gates))
        return ids, gates

    def rmsnorm(self, x, wnorm, eps):
        x = np.ascontiguousarray(x, dtype=np.float32)
        wnorm = np.ascontiguousarray(wnorm, dtype=np.float32)
        y = np.empty_like(x)
        self._rmsnorm(_ptr(wnorm), _ptr(x), _ptr(y), eps, x.size)
        return y

    def silu_mul(self, gate, up):
        gate = np.ascontiguousarray(gate, dtype=np.float32)
        up = np.ascontiguousarray(up, dtype=np.float32)
        h = np.empty_like(gate)
        self._silu_mul(_ptr(gate), _ptr(up), _ptr(h), gate.size)
        return h

    def wmerge(self, parts, gates, add1=None, add2=None, scale=1.0, n_full=0):
        parts = np.ascontiguousarray(parts, dtype=np.float32)
        n_parts, n = parts.shape
        g = None if gates is None else np.ascontiguousarray(gates, dtype=np.float32)
        a1 = None if add1 is None else np.ascontiguousarray(add1, dtype=np.float32)
        a2 = None if add2 is None else np.ascontiguousarray(add2, dtype=np.float32)
        y = np.empty(n, dtype=np.float32)
        self._wmerge(_ptr(parts), _ptr(g), _ptr(a1), _ptr(a2), _ptr(y), scale, n_parts, n, n_full)
        return y
