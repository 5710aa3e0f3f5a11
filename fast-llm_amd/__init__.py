"""Host-side mirror of the reference runtime's task interface over the HIP C-ABI.

The reference (qdox-labs/fast-llm) is C++17; its operator interface for this
path is the ``Task`` record with ``TaskKind`` / ``Fmt`` codes
(include/fastllm/fastllm.h:19-97) executed by ``exec_task_block`` /
``exec_task_cpu``.  This module binds ``include/fastllm_hip.h`` with ctypes
and exposes the same names and argument meanings, so parity tests read like
the reference's own tests.  It loads ONLY the in-tree ``libfastllm_hip.so``;
there is no CPU fallback: every op raises if the library or a GPU is absent.
"""
from __future__ import annotations

import ctypes as C
import enum
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libfastllm_hip.so")


class TaskKind(enum.IntEnum):
    """include/fastllm/fastllm.h:19-45 (stable numeric values)."""
    STREAM_DOT = 0
    MERGE = 1
    SIGNAL = 2
    ACT_Q8 = 3
    STREAM_DOT_IDX = 4
    RMSNORM = 5
    ADD2 = 6
    ROPE_DS2 = 7
    KV_APPEND = 8
    ATTN_HEAD = 9
    ROUTER_SEL = 10
    SILU_MUL = 11
    WMERGE = 12


class Fmt(enum.IntEnum):
    """include/fastllm/fastllm.h:56-57."""
    F32 = 0
    Q8_0 = 1
    Q5_0 = 2
    Q4_K = 3
    Q6_K = 4
    IQ2_XXS = 5
    IQ3_XXS = 6


BLK_ELEMS = {Fmt.F32: 1, Fmt.Q8_0: 32, Fmt.Q5_0: 32, Fmt.Q4_K: 256, Fmt.Q6_K: 256,
             Fmt.IQ2_XXS: 256, Fmt.IQ3_XXS: 256}
BLK_BYTES = {Fmt.F32: 4, Fmt.Q8_0: 34, Fmt.Q5_0: 22, Fmt.Q4_K: 144, Fmt.Q6_K: 210,
             Fmt.IQ2_XXS: 66, Fmt.IQ3_XXS: 98}
MAX_DOT_COLS = 16

OK, ERR_ARG, ERR_HIP, ERR_UNSUPPORTED, ERR_NOMEM, ERR_STATE, ERR_IO, ERR_FORMAT = \
    0, -1, -2, -3, -4, -5, -6, -7

# reference CPU default masks (src/runtime/kernels.h:920,937)
I8_MASK_DEFAULT = (1 << Fmt.Q8_0) | (1 << Fmt.Q5_0) | (1 << Fmt.Q4_K) | (1 << Fmt.Q6_K)
I8K_MASK_DEFAULT = (1 << Fmt.Q4_K) | (1 << Fmt.Q6_K)


def row_bytes(fmt: int, cols: int) -> int:
    """fl_row_bytes (src/runtime/quants.h:97-99)."""
    return (cols // BLK_ELEMS[Fmt(fmt)]) * BLK_BYTES[Fmt(fmt)]


def xq_offset(cols: int) -> int:
    """fl_xq_of offset (src/runtime/quants.h:302-304)."""
    return (cols * 4 + 15) & ~15


def xqk_offset(cols: int) -> int:
    """fl_xqk_of offset (src/runtime/quants.h:321-325)."""
    return xq_offset(cols) + (((cols // 32) * 36 + 15) & ~15)


def x_alloc_bytes(cols: int) -> int:
    """fl_x_alloc_bytes (src/runtime/quants.h:326-330)."""
    return xqk_offset(cols) + (cols // 256) * 292


class Task(C.Structure):
    """Byte layout of fastllm::Task (include/fastllm/fastllm.h:65-97)."""
    _fields_ = [
        ("id", C.c_uint32), ("kind", C.c_uint8), ("affinity", C.c_uint8),
        ("fmt", C.c_uint8), ("n_consumers", C.c_uint16),
        ("consumers", C.c_uint32 * 6), ("w", C.c_void_p), ("w_bytes", C.c_uint64),
        ("x", C.c_void_p), ("y", C.c_void_p), ("rows", C.c_uint32), ("cols", C.c_uint32),
        ("dep_init", C.c_int32), ("dep_count", C.c_int32), ("epoch", C.c_uint32),
        ("handoff_ts", C.c_uint64), ("aux", C.c_void_p), ("aux2", C.c_uint64),
        ("nx", C.c_uint32), ("xstride", C.c_uint32), ("ystride", C.c_uint32),
        ("_pad", C.c_uint8 * (256 - 132)),
    ]


class RmsNormP(C.Structure):
    """RmsNormP (src/runtime/decode_params.h:23-29)."""
    _fields_ = [("wnorm", C.c_void_p), ("x", C.c_void_p), ("y", C.c_void_p), ("eps", C.c_float),
                ("n", C.c_uint32)]


class RouterP(C.Structure):
    """RouterP (src/runtime/decode_params.h:68-75)."""
    _fields_ = [("logits", C.c_void_p), ("ids", C.c_void_p), ("gates", C.c_void_p),
                ("n_expert", C.c_uint32), ("top_k", C.c_uint32), ("norm", C.c_uint32),
                ("scale", C.c_float)]


class SiluMulP(C.Structure):
    """SiluMulP (src/runtime/decode_params.h:77-82)."""
    _fields_ = [("gate", C.c_void_p), ("up", C.c_void_p), ("h", C.c_void_p), ("n", C.c_uint32)]


class WmergeP(C.Structure):
    """WmergeP (src/runtime/decode_params.h:84-97)."""
    _fields_ = [("parts", C.c_void_p), ("gates", C.c_void_p), ("add1", C.c_void_p),
                ("add2", C.c_void_p), ("y", C.c_void_p), ("scale", C.c_float),
                ("n_parts", C.c_uint32), ("n", C.c_uint32), ("n_full", C.c_uint32)]


class GgufTensorInfo(C.Structure):
    """flh_gguf_tensor (GgufTensor, src/model/gguf.h:19-27)."""
    _fields_ = [("name", C.c_void_p), ("name_len", C.c_size_t), ("type", C.c_uint32),
                ("fmt", C.c_int32), ("n_dims", C.c_int32), ("ne", C.c_uint64 * 4),
                ("offset", C.c_uint64), ("nbytes", C.c_uint64), ("shard", C.c_int32),
                ("data", C.c_void_p)]


class WeightInfo(C.Structure):
    """flh_weight (WTensor as DecoderImpl::load_tensor fills it,
    src/model/decoder.cpp:186-206)."""
    _fields_ = [("fmt", C.c_int32), ("rows", C.c_uint32), ("cols", C.c_uint32),
                ("nexp", C.c_uint32), ("row_bytes", C.c_uint64), ("w_bytes", C.c_uint64),
                ("estride", C.c_uint64), ("host", C.c_void_p), ("tensor", C.c_uint64)]


class FlhError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"fastllm_hip error {code}: {msg}")
        self.code = code


_lib = None

_U32, _U64, _I, _P, _F, _SZ = C.c_uint32, C.c_uint64, C.c_int, C.c_void_p, C.c_float, C.c_size_t
_SIGS = {
    "flh_last_error": (C.c_char_p, []),
    "flh_init": (_I, [_I]),
    "flh_device_info": (_I, [C.POINTER(_I), C.POINTER(_SZ), C.POINTER(_I), C.c_char_p, _SZ]),
    "flh_default_masks": (None, [C.POINTER(_U32), C.POINTER(_U32)]),
    "flh_mfma_plan": (_I, [_U32, _U32, _U32, C.POINTER(_U32)]),
    "flh_row_bytes": (_U64, [_I, _U32]),
    "flh_x_alloc_bytes": (_SZ, [_U32]),
    "flh_arena_create": (_I, [_SZ, C.POINTER(_P)]),
    "flh_arena_alloc": (_I, [_P, _SZ, _SZ, C.POINTER(_P)]),
    "flh_arena_used": (_SZ, [_P]),
    "flh_arena_destroy": (_I, [_P]),
    "flh_malloc": (_I, [_SZ, C.POINTER(_P)]),
    "flh_free": (_I, [_P]),
    "flh_host_alloc": (_I, [_SZ, C.POINTER(_P)]),
    "flh_host_free": (_I, [_P]),
    "flh_upload": (_I, [_P, _P, _SZ, _P]),
    "flh_download": (_I, [_P, _P, _SZ, _P]),
    "flh_zero": (_I, [_P, _SZ, _P]),
    "flh_copy": (_I, [_P, _P, _SZ, _P]),
    "flh_stream_create": (_I, [C.POINTER(_P)]),
    "flh_stream_sync": (_I, [_P]),
    "flh_stream_destroy": (_I, [_P]),
    "flh_event_create": (_I, [C.POINTER(_P)]),
    "flh_event_record": (_I, [_P, _P]),
    "flh_event_elapsed_ms": (_I, [_P, _P, C.POINTER(_F)]),
    "flh_event_destroy": (_I, [_P]),
    "flh_graph_capture_begin": (_I, [_P]),
    "flh_graph_capture_end": (_I, [_P, C.POINTER(_P)]),
    "flh_graph_launch": (_I, [_P, _P]),
    "flh_graph_destroy": (_I, [_P]),
    "flh_act_q8": (_I, [_P, _P, _U32, _U32, _U32, _P]),
    "flh_stream_dot": (_I, [_I, _P, _U64, _U32, _U32, _P, _P, _U32, _U32, _U32, _P, _U64,
                            _I, _U32, _U32, _P]),
    "flh_act_q8_stream_dot": (_I, [_I, _P, _U64, _U32, _U32, _P, _P, _U32, _U32, _U32, _P, _U64,
                                   _I, _U32, _U32, _P]),
    "flh_exec_tasks": (_I, [_P, _U32, _I, _U32, _U32, _P]),
    "flh_dequant": (_I, [_I, _P, _U32, _U32, _P, _P]),
    "flh_moe_dot": (_I, [_I, _P, _U64, _U32, _U32, _P, _U32, _U32, _U32, _P, _U32, _U32, _P,
                         _U32, _P]),
    "flh_router_sel": (_I, [_P, _U32, _U32, _U32, _U32, _F, _P, _P, _P]),
    "flh_router_moe_dot": (_I, [_I, _P, _U64, _U32, _U32, _P, _U32, _U32, _U32, _U32, _F, _P, _P, _P,
                                _U32, _U32, _P, _U32, _P]),
    "flh_silu_mul": (_I, [_P, _P, _P, _U32, _U32, _U32, _U32, _P]),
    "flh_silu_mul_act_q8": (_I, [_P, _P, _P, _U32, _U32, _U32, _U32, _P]),
    "flh_rmsnorm_act_q8": (_I, [_P, _P, _P, _U32, C.c_float, _I, _P]),
    "flh_rmsnorm_stream_dot": (_I, [_I, _P, _U64, _U32, _U32, _P, _P, C.c_float, _P, _P, _I, _U32, _U32, _P]),
    "flh_wmerge": (_I, [_P, _P, _P, _P, _P, _F, _U32, _U32, _U32, _U32, _U32, _U32, _P]),
    "flh_fill_normal": (_I, [_P, _SZ, _U64, _F, _F, _F, _F, _P]),
    "flh_quantize": (_I, [_I, _P, _U32, _U32, _P, _P]),
    "flh_quantize_host": (_I, [_I, _P, _U32, _U32, _P]),
    "flh_gguf_open": (_I, [C.c_char_p, C.POINTER(_P)]),
    "flh_gguf_close": (_I, [_P]),
    "flh_gguf_alignment": (_U32, [_P]),
    "flh_gguf_n_shards": (_I, [_P]),
    "flh_gguf_n_tensors": (_U64, [_P]),
    "flh_gguf_tensor_info": (_I, [_P, _U64, C.POINTER(GgufTensorInfo)]),
    "flh_gguf_find": (C.c_int64, [_P, C.c_char_p]),
    "flh_gguf_fmt_of": (_I, [_U32]),
    "flh_gguf_type_name": (C.c_char_p, [_U32]),
    "flh_gguf_has": (_I, [_P, C.c_char_p]),
    "flh_gguf_kv_i": (C.c_int64, [_P, C.c_char_p, C.c_int64]),
    "flh_gguf_kv_f": (C.c_double, [_P, C.c_char_p, C.c_double]),
    "flh_gguf_kv_s": (_P, [_P, C.c_char_p, C.c_char_p, C.POINTER(_SZ)]),
    "flh_gguf_kv_sarr_len": (C.c_int64, [_P, C.c_char_p]),
    "flh_gguf_kv_sarr_at": (_P, [_P, C.c_char_p, _U64, C.POINTER(_SZ)]),
    "flh_gguf_weight": (_I, [_P, C.c_char_p, C.POINTER(WeightInfo)]),
    "flh_gguf_upload": (_I, [_P, _U64, _P, _U64, _P]),
    "flh_gguf_upload_all": (_I, [_P, _P, C.POINTER(_P), _P]),
}


def lib():
    """Load the in-tree HIP library (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FlhError(ERR_STATE, f"{LIB_PATH} not built: run __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != OK:
        raise FlhError(rc, lib().flh_last_error().decode())


def _p(v):
    """Device pointer argument: DeviceBuffer, int address or None."""
    if v is None:
        return None
    if isinstance(v, DeviceBuffer):
        return v.ptr
    return int(v)


_initialised = False


def init(device: int = 0) -> None:
    global _initialised
    check(lib().flh_init(device))
    _initialised = True


def device_info() -> dict:
    cus, hbm, ws = C.c_int(), C.c_size_t(), C.c_int()
    name = C.create_string_buffer(128)
    check(lib().flh_device_info(C.byref(cus), C.byref(hbm), C.byref(ws), name, 128))
    return {"num_cus": cus.value, "hbm_bytes": hbm.value, "wave_size": ws.value,
            "arch": name.value.decode()}


def mfma_plan(rows: int, cols: int, nx: int):
    """The multi-column matrix-core kernel's plan for a Q4_K rows x cols
    matrix with nx columns: {"kh", "xc", "nrb", "D"}, or None when that kernel
    does not take the shape."""
    out = (_U32 * 4)()
    rc = lib().flh_mfma_plan(rows, cols, nx, out)
    if rc == ERR_UNSUPPORTED:
        return None
    check(rc)
    return {"kh": bool(out[0]), "xc": bool(out[1]), "nrb": out[2], "D": out[3]}


class Stream:
    def __init__(self):
        h = C.c_void_p()
        check(lib().flh_stream_create(C.byref(h)))
        self.handle = h.value

    def sync(self):
        check(lib().flh_stream_sync(self.handle))

    def close(self):
        if self.handle:
            check(lib().flh_stream_destroy(self.handle))
            self.handle = None


class Event:
    def __init__(self):
        h = C.c_void_p()
        check(lib().flh_event_create(C.byref(h)))
        self.handle = h.value

    def record(self, stream: Stream):
        check(lib().flh_event_record(self.handle, stream.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        check(lib().flh_event_elapsed_ms(self.handle, end.handle, C.byref(ms)))
        return ms.value

    def close(self):
        if self.handle:
            check(lib().flh_event_destroy(self.handle))
            self.handle = None


class Graph:
    """A captured HIP graph: `with Graph.capture(stream) as g: <issue work>`."""

    def __init__(self, stream: Stream):
        self.stream = stream
        self.handle = None

    @classmethod
    def capture(cls, stream: Stream) -> "Graph":
        return cls(stream)

    def __enter__(self):
        check(lib().flh_graph_capture_begin(self.stream.handle))
        return self

    def __exit__(self, et, ev, tb):
        h = C.c_void_p()
        rc = lib().flh_graph_capture_end(self.stream.handle, C.byref(h))
        if et is None:
            check(rc)
            self.handle = h.value
        return False

    def launch(self, stream: Stream | None = None) -> None:
        check(lib().flh_graph_launch(self.handle, (stream or self.stream).handle))

    def close(self):
        if self.handle:
            check(lib().flh_graph_destroy(self.handle))
            self.handle = None


class HostBuffer:
    """Pinned host memory (flh_host_alloc): host-readable and device-visible,
    the place for decode-op param blocks of a task table.  `view(ctype)`
    gives a ctypes object over its first bytes."""

    def __init__(self, nbytes: int):
        h = C.c_void_p()
        check(lib().flh_host_alloc(max(int(nbytes), 1), C.byref(h)))
        self.ptr = h.value
        self.nbytes = int(nbytes)

    def view(self, ctype):
        assert C.sizeof(ctype) <= self.nbytes
        return ctype.from_address(self.ptr)

    def close(self):
        if self.ptr and lib():
            lib().flh_host_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DeviceBuffer:
    """A hipMalloc'd device buffer (freed on close / garbage collection)."""

    def __init__(self, nbytes: int):
        h = C.c_void_p()
        check(lib().flh_malloc(max(int(nbytes), 1), C.byref(h)))
        self.ptr = h.value
        self.nbytes = int(nbytes)

    @classmethod
    def from_array(cls, arr: np.ndarray, stream: Stream, extra: int = 0) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        b = cls(arr.nbytes + extra)
        b.upload(arr, stream)
        return b

    def upload(self, arr: np.ndarray, stream: Stream, offset: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        assert offset + arr.nbytes <= self.nbytes
        check(lib().flh_upload(self.ptr + offset, arr.ctypes.data, arr.nbytes, stream.handle))

    def download(self, dtype, count: int, stream: Stream, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        check(lib().flh_download(out.ctypes.data, self.ptr + offset, out.nbytes, stream.handle))
        return out

    def zero(self, stream: Stream) -> None:
        check(lib().flh_zero(self.ptr, self.nbytes, stream.handle))

    def close(self):
        if self.ptr and lib():
            lib().flh_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---------------------------------------------------------------- ops --
def copy(dst, src, n: int, stream: Stream) -> None:
    check(lib().flh_copy(_p(dst), _p(src), n, stream.handle))


def act_q8(x, cols: int, stream: Stream, nx: int = 1, xstride: int = 0, y_q81=None) -> None:
    """ACT_Q8 (fl_exec_act_q8, src/runtime/quants.h:404-416) on nx columns."""
    check(lib().flh_act_q8(_p(x), _p(y_q81), cols, nx, xstride, stream.handle))


def stream_dot(fmt: int, w, rows: int, cols: int, x, y, stream: Stream, nx: int = 1,
               xstride: int = 0, ystride: int = 0, id_slot=None, estride: int = 0,
               fast: bool = True, i8_mask: int = I8_MASK_DEFAULT,
               i8k_mask: int = I8K_MASK_DEFAULT, w_bytes: int | None = None) -> None:
    """One STREAM_DOT / STREAM_DOT_IDX tile (exec_task_cpu semantics, y +=)."""
    if w_bytes is None:
        w_bytes = rows * row_bytes(fmt, cols)
    check(lib().flh_stream_dot(int(fmt), _p(w), w_bytes, rows, cols, _p(x), _p(y), nx,
                               xstride, ystride, _p(id_slot), estride, int(bool(fast)),
                               i8_mask, i8k_mask, stream.handle))


def act_q8_stream_dot(fmt: int, w, rows: int, cols: int, x, y, stream: Stream, nx: int = 1,
                      xstride: int = 0, ystride: int = 0, id_slot=None, estride: int = 0,
                      fast: bool = True, i8_mask: int = I8_MASK_DEFAULT,
                      i8k_mask: int = I8K_MASK_DEFAULT) -> None:
    """ACT_Q8 + STREAM_DOT on the same activation (fused where possible)."""
    w_bytes = rows * row_bytes(fmt, cols)
    check(lib().flh_act_q8_stream_dot(int(fmt), _p(w), w_bytes, rows, cols, _p(x), _p(y), nx,
                                      xstride, ystride, _p(id_slot), estride, int(bool(fast)),
                                      i8_mask, i8k_mask, stream.handle))


def exec_tasks(tasks, stream: Stream, fast: bool = True, i8_mask: int = I8_MASK_DEFAULT,
               i8k_mask: int = I8K_MASK_DEFAULT) -> None:
    """Run a task table in order (the executor's per-task dispatch)."""
    arr = (Task * len(tasks))(*tasks)
    check(lib().flh_exec_tasks(C.cast(arr, C.c_void_p), len(tasks), int(bool(fast)),
                               i8_mask, i8k_mask, stream.handle))


def dequant(fmt: int, w, rows: int, cols: int, out, stream: Stream) -> None:
    check(lib().flh_dequant(int(fmt), _p(w), rows, cols, _p(out), stream.handle))


def moe_dot(fmt: int, w, estride: int, rows: int, cols: int, ids, ntok: int, top_k: int,
            n_expert: int, x, xstride: int, x_per_slot: bool, y, ystride: int,
            stream: Stream) -> None:
    check(lib().flh_moe_dot(int(fmt), _p(w), estride, rows, cols, _p(ids), ntok, top_k,
                            n_expert, _p(x), xstride, int(bool(x_per_slot)), _p(y), ystride,
                            stream.handle))


def router_moe_dot(fmt: int, w, estride: int, rows: int, cols: int, logits, ntok: int, n_expert: int,
                   top_k: int, norm: int, scale: float, ids, gates, x, xstride: int, x_per_slot: bool, y,
                   ystride: int, stream: Stream) -> None:
    """ROUTER_SEL + grouped expert matvec in one launch (same bits as router_sel then moe_dot)."""
    check(lib().flh_router_moe_dot(int(fmt), _p(w), estride, rows, cols, _p(logits), ntok, n_expert, top_k,
                                   norm, scale, _p(ids), _p(gates), _p(x), xstride, int(bool(x_per_slot)),
                                   _p(y), ystride, stream.handle))


def router_sel(logits, ntok, n_expert, top_k, norm, scale, ids, gates, stream: Stream):
    check(lib().flh_router_sel(_p(logits), ntok, n_expert, top_k, norm, scale, _p(ids),
                               _p(gates), stream.handle))


def silu_mul(gate, up, h, n, ncol, gstride, hstride, stream: Stream):
    check(lib().flh_silu_mul(_p(gate), _p(up), _p(h), n, ncol, gstride, hstride, stream.handle))


def silu_mul_act_q8(gate, up, h, n, ncol, gstride, hstride, stream: Stream):
    """SILU_MUL then ACT_Q8 of every h column (one launch, same bytes)."""
    check(lib().flh_silu_mul_act_q8(_p(gate), _p(up), _p(h), n, ncol, gstride, hstride, stream.handle))


def rmsnorm_act_q8(x, wnorm, y, n, eps, stream: Stream, write_app: bool = True):
    """RMSNORM of one column (y = x * s * wnorm) and, with write_app, the
    ACT_Q8 appendices of y, in one launch."""
    check(lib().flh_rmsnorm_act_q8(_p(x), _p(wnorm), _p(y), n, eps, int(bool(write_app)), stream.handle))


def rmsnorm_stream_dot(fmt: int, w, rows: int, cols: int, x, wnorm, eps: float, xn, y, stream: Stream,
                       fast: bool = True, i8_mask: int = I8_MASK_DEFAULT,
                       i8k_mask: int = I8K_MASK_DEFAULT) -> None:
    """RMSNORM of x into xn (with its ACT_Q8 appendices), then y += W xn
    (one launch where the kernel takes it; the bits of rmsnorm_act_q8 followed
    by stream_dot either way)."""
    w_bytes = rows * row_bytes(fmt, cols)
    check(lib().flh_rmsnorm_stream_dot(int(fmt), _p(w), w_bytes, rows, cols, _p(x), _p(wnorm), eps, _p(xn),
                                       _p(y), int(bool(fast)), i8_mask, i8k_mask, stream.handle))


def wmerge(parts, gates, add1, add2, y, scale, n_parts, n, n_full, ncol, pstride, ystride,
           stream: Stream):
    check(lib().flh_wmerge(_p(parts), _p(gates), _p(add1), _p(add2), _p(y), scale, n_parts, n,
                           n_full, ncol, pstride, ystride, stream.handle))


def fill_normal(dst, n: int, seed: int, stream: Stream, mean: float = 0.0, std: float = 1.0,
                outlier_frac: float = 0.0, outlier_scale: float = 1.0) -> None:
    check(lib().flh_fill_normal(_p(dst), n, seed, mean, std, outlier_frac, outlier_scale,
                                stream.handle))


def quantize(fmt: int, src, rows: int, cols: int, dst, stream: Stream) -> None:
    check(lib().flh_quantize(int(fmt), _p(src), rows, cols, _p(dst), stream.handle))


def quantize_host(fmt: int, w: np.ndarray) -> np.ndarray:
    """fp32 [rows, cols] -> block bytes, same bytes as the device quantizer."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    out = np.zeros(rows * row_bytes(fmt, cols), dtype=np.uint8)
    check(lib().flh_quantize_host(int(fmt), w.ctypes.data, rows, cols, out.ctypes.data))
    return out


# --------------------------------------------------------------- arena --
class Arena:
    """Device bump arena (flh_arena_*; Arena, src/runtime/arena.cpp:54-74)."""

    def __init__(self, nbytes: int):
        h = C.c_void_p()
        check(lib().flh_arena_create(int(nbytes), C.byref(h)))
        self.handle = h.value

    def alloc(self, nbytes: int, align: int = 256) -> int:
        p = C.c_void_p()
        check(lib().flh_arena_alloc(self.handle, int(nbytes), int(align), C.byref(p)))
        return p.value

    @property
    def used(self) -> int:
        return lib().flh_arena_used(self.handle)

    def close(self):
        if self.handle:
            check(lib().flh_arena_destroy(self.handle))
            self.handle = None


# ---------------------------------------------------------------- GGUF --
class GgufTensor:
    """One tensor info; `data` is a read-only uint8 view of the mapping."""

    def __init__(self, g: "Gguf", index: int, ti: GgufTensorInfo):
        self.index = index
        self.name = C.string_at(ti.name, ti.name_len).decode("utf-8", "surrogateescape")
        self.type = ti.type
        self.fmt = ti.fmt
        self.n_dims = ti.n_dims
        self.ne = tuple(ti.ne)
        self.offset = ti.offset
        self.nbytes = ti.nbytes
        self.shard = ti.shard
        self.address = ti.data
        self._g = g

    @property
    def data(self) -> np.ndarray:
        if self.nbytes == 0:
            return np.zeros(0, dtype=np.uint8)
        buf = (C.c_uint8 * self.nbytes).from_address(self.address)
        a = np.frombuffer(buf, dtype=np.uint8)
        a.flags.writeable = False
        return a


class Gguf:
    """GGUF reader over the C-ABI (fastllm::Gguf, src/model/gguf.h:28-79).

    Same method names as the reference: open (the constructor), tensors,
    find, data, alignment, n_shards, has, kv_i, kv_f, kv_s, kv_sarr, fmt_of,
    type_name.  Errors raise FlhError (ERR_IO for a missing file or shard,
    ERR_FORMAT for a malformed one) where the reference returns false or
    aborts.  Parsing is host-only; upload / upload_all copy to the device.
    """

    def __init__(self, path: str):
        h = C.c_void_p()
        check(lib().flh_gguf_open(os.fsencode(path), C.byref(h)))
        self.handle = h.value
        L = lib()
        self._tensors = []
        for i in range(L.flh_gguf_n_tensors(self.handle)):
            ti = GgufTensorInfo()
            check(L.flh_gguf_tensor_info(self.handle, i, C.byref(ti)))
            self._tensors.append(GgufTensor(self, i, ti))

    def close(self):
        if self.handle:
            lib().flh_gguf_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()
        return False

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensors(self) -> list:
        return list(self._tensors)

    def find(self, name: str) -> GgufTensor | None:
        i = lib().flh_gguf_find(self.handle, name.encode("utf-8", "surrogateescape"))
        return None if i < 0 else self._tensors[i]

    def data(self, t: GgufTensor) -> np.ndarray:
        return t.data

    def alignment(self) -> int:
        return lib().flh_gguf_alignment(self.handle)

    def n_shards(self) -> int:
        return lib().flh_gguf_n_shards(self.handle)

    def has(self, key: str) -> bool:
        return bool(lib().flh_gguf_has(self.handle, key.encode("utf-8", "surrogateescape")))

    def kv_i(self, key: str, dflt: int) -> int:
        return lib().flh_gguf_kv_i(self.handle, key.encode("utf-8", "surrogateescape"), int(dflt))

    def kv_f(self, key: str, dflt: float) -> float:
        return lib().flh_gguf_kv_f(self.handle, key.encode("utf-8", "surrogateescape"), float(dflt))

    def kv_s(self, key: str, dflt: str = "") -> str:
        n = C.c_size_t()
        p = lib().flh_gguf_kv_s(self.handle, key.encode("utf-8", "surrogateescape"), dflt.encode(), C.byref(n))
        return C.string_at(p, n.value).decode("utf-8", "surrogateescape")

    def kv_sarr(self, key: str) -> list | None:
        L = lib()
        n = L.flh_gguf_kv_sarr_len(self.handle, key.encode("utf-8", "surrogateescape"))
        if n < 0:
            return None
        out, ln = [], C.c_size_t()
        for i in range(n):
            p = L.flh_gguf_kv_sarr_at(self.handle, key.encode("utf-8", "surrogateescape"), i, C.byref(ln))
            out.append(C.string_at(p, ln.value).decode("utf-8", "surrogateescape"))
        return out

    @staticmethod
    def fmt_of(ggml_type: int) -> int | None:
        f = lib().flh_gguf_fmt_of(ggml_type)
        return None if f < 0 else f

    @staticmethod
    def type_name(ggml_type: int) -> str:
        return lib().flh_gguf_type_name(ggml_type).decode()

    def weight(self, name: str) -> WeightInfo:
        w = WeightInfo()
        check(lib().flh_gguf_weight(self.handle, name.encode("utf-8", "surrogateescape"), C.byref(w)))
        return w

    def upload(self, t: GgufTensor, dst, stream: Stream, dst_bytes: int | None = None) -> None:
        n = t.nbytes if dst_bytes is None else dst_bytes
        check(lib().flh_gguf_upload(self.handle, t.index, _p(dst), n, stream.handle))

    def upload_all(self, arena: Arena, stream: Stream) -> list:
        """Device pointer per tensor (None where the payload size is unknown)."""
        n = len(self._tensors)
        ptrs = (C.c_void_p * max(n, 1))()
        check(lib().flh_gguf_upload_all(self.handle, arena.handle, ptrs, stream.handle))
        return [ptrs[i] for i in range(n)]
