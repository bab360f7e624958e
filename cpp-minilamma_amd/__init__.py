"""Python binding of libminilamma_hip.so (the C ABI in include/minilamma_hip.h).

The binding is ctypes over the C ABI and nothing else: no torch, no CPU
fallback.  Importing it on a machine where the library was not built raises
ImportError; calling an op without a GPU raises MlkError from the HIP
runtime.  Device memory is held by DeviceBuffer (hipMalloc through the ABI);
host arrays are numpy.

The directory name is not a Python identifier, so callers load this file with
`load_package()` from __graft_entry__.py (or importlib) under the module name
`cpp_minilamma_amd`.

Op wrappers mirror the reference's operator surface (include/cuda_ops.h):
the same argument meaning and the same rejections, raised as MlkError whose
text carries the caller name, like the reference's std::runtime_error
"<Caller>: <reason>" messages.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "lib")
HIP_LIB = os.path.join(LIB_DIR, "libminilamma_hip.so")
OPS_LIB = os.path.join(LIB_DIR, "libminilamma_ops.so")

MLK_OK, MLK_ERR_INVALID, MLK_ERR_RANGE, MLK_ERR_HIP, MLK_ERR_NO_DEVICE = range(5)
ROPE_NORMAL, ROPE_NEOX = 0, 1
QUANT = {"q8_0": 0, "q4_0": 1, "q4_1": 2}
BLOCK_BYTES = {"q8_0": 34, "q4_0": 18, "q4_1": 20}
H2D, D2D, D2H = 0, 1, 2


class MlkError(RuntimeError):
    def __init__(self, status, message):
        super().__init__(message)
        self.status = status


class DeviceInfo(C.Structure):
    _fields_ = [("device_id", C.c_int), ("name", C.c_char * 256), ("arch", C.c_char * 64),
                ("compute_major", C.c_int), ("compute_minor", C.c_int),
                ("total_bytes", C.c_size_t), ("multiprocessors", C.c_int),
                ("clock_khz", C.c_int), ("memory_clock_khz", C.c_int),
                ("memory_bus_bits", C.c_int), ("runtime_version", C.c_int),
                ("driver_version", C.c_int)]


_vp = C.c_void_p
_i64 = C.c_int64
_i32 = C.c_int32
_f = C.c_float

# name -> argtypes; every op returns mlk_status (int)
_SIGNATURES = {
    "mlk_add_rmsnorm_f32": [_vp, _vp, _vp, _vp, _i64, _i64, _f, _vp],
    "mlk_rmsnorm_f32": [_vp, _vp, _vp, _i64, _i64, _f, _vp],
    "mlk_swiglu_f32": [_vp, _vp, _vp, _i64, _vp],
    "mlk_silu_f32": [_vp, _vp, _i64, _vp],
    "mlk_mul_f32": [_vp, _vp, _vp, _i64, _vp],
    "mlk_add_f32": [_vp, _vp, _vp, _i64, _vp],
    "mlk_softmax_f32": [_vp, _vp, _i64, _i64, _vp],
    "mlk_rope_f32": [_vp, _vp, _i64, _i32, _i32, _i32, _i64, _i64, _vp, _i32, _f, _i32, _vp, _vp],
    "mlk_gather_f32": [_vp, _i64, _i64, _vp, _i32, _i64, _vp, _vp, _vp],
    "mlk_gather_quant": [_i32, _vp, _i64, _i64, _vp, _i32, _i64, _vp, _vp, _vp],
    "mlk_quantize": [_i32, _vp, _i64, _i64, _vp, _vp],
    "mlk_linear_quant": [_i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, C.c_size_t, _vp],
    "mlk_linear_f32": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, C.c_size_t, _vp],
    "mlk_quant_to_planar": [_i32, _vp, _i64, _i64, _vp, _vp],
    "mlk_linear_planar": [_i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, C.c_size_t, _vp],
    "mlk_matmul_f32": [_vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "mlk_fill_normal_f32": [_vp, _i64, _f, _f, C.c_uint64, _vp],
    "mlk_kv_write_f32": [_vp, _vp, _i64, _i64, _i32, _i32, _i64, _vp, _i64, _vp, _i64, _vp, _i32,
                         _i64, _vp, _vp],
    "mlk_attention_decode_f32": [_vp, _i64, _vp, _vp, _i64, _i64, _i32, _i32, _i32, _i64, _vp,
                                 _i32, _i64, _i64, _vp, _vp, C.c_size_t, _vp, _vp],
    "mlk_attention_prefill_f32": [_vp, _i64, _vp, _vp, _i64, _i64, _i32, _i32, _i32, _i64, _i32,
                                  _i64, _vp, _vp],
    "mlk_attention_decode_f32_noalloc": [_vp, _i64, _vp, _vp, _i64, _i64, _i32, _i32, _i32, _i64,
                                         _vp, _i32, _i64, _i64, _vp, _vp, _vp],
    "mlk_device_count": [C.POINTER(C.c_int)],
    "mlk_set_device": [C.c_int],
    "mlk_get_device": [C.POINTER(C.c_int)],
    "mlk_get_device_info": [C.c_int, C.POINTER(DeviceInfo)],
    "mlk_malloc": [C.POINTER(_vp), C.c_size_t],
    "mlk_free": [_vp],
    "mlk_memcpy": [_vp, _vp, C.c_size_t, _i32],
    "mlk_memcpy_async": [_vp, _vp, C.c_size_t, _i32, _vp],
    "mlk_zero_async": [_vp, C.c_size_t, _vp],
    "mlk_device_synchronize": [],
    "mlk_stream_create": [C.POINTER(_vp)],
    "mlk_stream_destroy": [_vp],
    "mlk_stream_synchronize": [_vp],
    "mlk_event_create": [C.POINTER(_vp)],
    "mlk_event_destroy": [_vp],
    "mlk_event_record": [_vp, _vp],
    "mlk_event_synchronize": [_vp],
    "mlk_event_elapsed_ms": [C.POINTER(_f), _vp, _vp],
    "mlk_graph_begin_capture": [_vp],
    "mlk_graph_end_capture": [_vp, C.POINTER(_vp)],
    "mlk_graph_launch": [_vp, _vp],
    "mlk_graph_destroy": [_vp],
}


def _load():
    if not os.path.exists(HIP_LIB):
        raise ImportError(
            f"{HIP_LIB} is missing: build it with `python -c 'import __graft_entry__ as g; "
            "g.build()'` (hipcc, gfx950). There is no CPU fallback.")
    lib = C.CDLL(HIP_LIB)
    for name, args in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = C.c_int
    lib.mlk_last_error.restype = C.c_char_p
    lib.mlk_last_error.argtypes = []
    lib.mlk_status_string.restype = C.c_char_p
    lib.mlk_status_string.argtypes = [C.c_int]
    lib.mlk_abi_version.restype = C.c_int
    lib.mlk_abi_version.argtypes = []
    lib.mlk_quant_bytes.restype = C.c_int64
    lib.mlk_quant_bytes.argtypes = [_i32, _i64, _i64]
    lib.mlk_attention_workspace_bytes.restype = C.c_int64
    lib.mlk_attention_workspace_bytes.argtypes = [_i64, _i32, _i32, _i32, _i64]
    lib.mlk_attention_noalloc_scratch_bytes.restype = C.c_size_t
    lib.mlk_attention_noalloc_scratch_bytes.argtypes = []
    lib.mlk_linear_workspace_bytes.restype = C.c_int64
    lib.mlk_linear_workspace_bytes.argtypes = [_i64, _i64, _i64]
    lib.mlk_quant_planar_bytes.restype = C.c_int64
    lib.mlk_quant_planar_bytes.argtypes = [_i32, _i64, _i64]
    lib.mlk_linear_planar_workspace_bytes.restype = C.c_int64
    lib.mlk_linear_planar_workspace_bytes.argtypes = [_i64, _i64, _i64]
    return lib


lib = _load()


def check(status, caller=None):
    if status != MLK_OK:
        msg = lib.mlk_last_error().decode(errors="replace")
        if caller and not msg.startswith(caller):
            msg = f"{caller}: {msg}"
        raise MlkError(status, msg)


def exported_symbols():
    """Names of every C ABI function the binding binds (used by the CPU tests)."""
    return sorted(list(_SIGNATURES) + ["mlk_last_error", "mlk_status_string",
                                       "mlk_abi_version", "mlk_quant_bytes",
                                       "mlk_attention_workspace_bytes",
                                       "mlk_linear_workspace_bytes",
                                       "mlk_quant_planar_bytes",
                                       "mlk_linear_planar_workspace_bytes",
                                       # bound with their structs in forward.py
                                       "mlk_forward_layer_workspace_bytes",
                                       "mlk_forward_layer_batch"])


# ------------------------------------------------------------------ runtime

def device_count():
    n = C.c_int(0)
    check(lib.mlk_device_count(C.byref(n)))
    return n.value


def set_device(device_id):
    check(lib.mlk_set_device(device_id))


def device_info(device_id=0):
    info = DeviceInfo()
    check(lib.mlk_get_device_info(device_id, C.byref(info)))
    arch = info.arch.decode()
    # the runtime leaves the marketing name empty on some boxes: fall back to
    # the architecture name, as GetCudaInfo does
    return {"name": info.name.decode() or arch, "arch": arch,
            "compute_units": info.multiprocessors, "total_bytes": info.total_bytes,
            "clock_khz": info.clock_khz, "memory_clock_khz": info.memory_clock_khz,
            "memory_bus_bits": info.memory_bus_bits, "runtime_version": info.runtime_version,
            "driver_version": info.driver_version}


def synchronize():
    check(lib.mlk_device_synchronize())


class DeviceBuffer:
    """A device allocation of `nbytes` (hipMalloc), freed on close/GC."""

    def __init__(self, nbytes, dtype=np.float32, shape=None):
        self.nbytes = int(nbytes)
        self.dtype = np.dtype(dtype)
        self.shape = tuple(shape) if shape is not None else (self.nbytes // self.dtype.itemsize,)
        p = _vp()
        check(lib.mlk_malloc(C.byref(p), self.nbytes), "DeviceBuffer")
        self.ptr = p.value or 0

    @classmethod
    def empty(cls, shape, dtype=np.float32):
        shape = tuple(int(s) for s in np.atleast_1d(shape))
        dt = np.dtype(dtype)
        return cls(int(np.prod(shape)) * dt.itemsize, dt, shape)

    @classmethod
    def from_array(cls, arr):
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes, arr.dtype, arr.shape)
        buf.upload(arr)
        return buf

    def upload(self, arr):
        arr = np.ascontiguousarray(arr, dtype=self.dtype)
        if arr.nbytes > self.nbytes:
            raise ValueError("upload exceeds device buffer size")
        check(lib.mlk_memcpy(self.ptr, arr.ctypes.data, arr.nbytes, H2D), "upload")

    def download(self, shape=None, dtype=None):
        dt = np.dtype(dtype) if dtype is not None else self.dtype
        shape = tuple(shape) if shape is not None else (
            self.shape if dt == self.dtype else (self.nbytes // dt.itemsize,))
        out = np.empty(shape, dtype=dt)
        if out.nbytes > self.nbytes:
            raise ValueError("download exceeds device buffer size")
        check(lib.mlk_memcpy(out.ctypes.data, self.ptr, out.nbytes, D2H), "download")
        return out

    def zero(self, stream=None):
        check(lib.mlk_zero_async(self.ptr, self.nbytes, _sp(stream)), "zero")

    def offset(self, nbytes):
        """Raw device address nbytes into the buffer (for sub-views)."""
        return self.ptr + int(nbytes)

    def close(self):
        if getattr(self, "ptr", 0):
            lib.mlk_free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __int__(self):
        return self.ptr


class Stream:
    def __init__(self):
        s = _vp()
        check(lib.mlk_stream_create(C.byref(s)), "Stream")
        self.handle = s.value

    def synchronize(self):
        check(lib.mlk_stream_synchronize(self.handle), "Stream.synchronize")

    def close(self):
        if self.handle:
            lib.mlk_stream_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Event:
    def __init__(self):
        e = _vp()
        check(lib.mlk_event_create(C.byref(e)), "Event")
        self.handle = e.value

    def record(self, stream=None):
        check(lib.mlk_event_record(self.handle, _sp(stream)), "Event.record")

    def synchronize(self):
        check(lib.mlk_event_synchronize(self.handle), "Event.synchronize")

    def elapsed_ms(self, end):
        ms = _f(0.0)
        check(lib.mlk_event_elapsed_ms(C.byref(ms), self.handle, end.handle), "Event.elapsed_ms")
        return ms.value

    def close(self):
        if self.handle:
            lib.mlk_event_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Graph:
    """An executable HIP graph captured from the ops issued on `stream`
    inside `with Graph.capture(stream) as g:`; replay with g.launch()."""

    def __init__(self, stream):
        self.stream = stream
        self.handle = None

    @classmethod
    def capture(cls, stream):
        return _Capture(cls(stream))

    def launch(self, stream=None):
        check(lib.mlk_graph_launch(self.handle, _sp(stream or self.stream)), "Graph.launch")

    def close(self):
        if self.handle:
            lib.mlk_graph_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class _Capture:
    def __init__(self, graph):
        self.graph = graph

    def __enter__(self):
        check(lib.mlk_graph_begin_capture(_sp(self.graph.stream)), "Graph.capture")
        return self.graph

    def __exit__(self, exc_type, exc, tb):
        h = _vp()
        st = lib.mlk_graph_end_capture(_sp(self.graph.stream), C.byref(h))
        self.graph.handle = h.value
        if exc_type is None:
            check(st, "Graph.capture")
        return False


def _sp(stream):
    if stream is None:
        return None
    return stream.handle if isinstance(stream, Stream) else stream


def _p(x):
    """Device address of a DeviceBuffer / int / None."""
    if x is None:
        return None
    return x.ptr if isinstance(x, DeviceBuffer) else int(x)


# ---------------------------------------------------------------------- ops

def add_rmsnorm(residual, delta, weight, y, n_rows, dim, eps, stream=None):
    """residual <- residual + delta; y <- RMSNorm(residual) * weight (row-wise)."""
    check(lib.mlk_add_rmsnorm_f32(_p(residual), _p(delta), _p(weight), _p(y), n_rows, dim, eps,
                                  _sp(stream)), "mlk_add_rmsnorm_f32")


def rmsnorm(x, weight, y, n_rows, dim, eps, stream=None):
    check(lib.mlk_rmsnorm_f32(_p(x), _p(weight), _p(y), n_rows, dim, eps, _sp(stream)),
          "mlk_rmsnorm_f32")


def swiglu(gate, up, y, n, stream=None):
    check(lib.mlk_swiglu_f32(_p(gate), _p(up), _p(y), n, _sp(stream)), "mlk_swiglu_f32")


def silu(x, y, n, stream=None):
    check(lib.mlk_silu_f32(_p(x), _p(y), n, _sp(stream)), "mlk_silu_f32")


def mul(a, b, y, n, stream=None):
    check(lib.mlk_mul_f32(_p(a), _p(b), _p(y), n, _sp(stream)), "mlk_mul_f32")


def add(a, b, y, n, stream=None):
    check(lib.mlk_add_f32(_p(a), _p(b), _p(y), n, _sp(stream)), "mlk_add_f32")


def softmax(x, y, n_rows, n, stream=None):
    check(lib.mlk_softmax_f32(_p(x), _p(y), n_rows, n, _sp(stream)), "mlk_softmax_f32")


def rope(q, k, n_tokens, n_heads, n_kv_heads, head_dim, positions=None, pos0=0, theta=10000.0,
         rope_type=ROPE_NORMAL, q_row_stride=None, k_row_stride=None, err=None, stream=None):
    qs = q_row_stride if q_row_stride is not None else n_heads * head_dim
    ks = k_row_stride if k_row_stride is not None else n_kv_heads * head_dim
    check(lib.mlk_rope_f32(_p(q), _p(k), n_tokens, n_heads, n_kv_heads, head_dim, qs, ks,
                           _p(positions), pos0, theta, rope_type, _p(err), _sp(stream)),
          "mlk_rope_f32")


def gather_f32(table, vocab, dim, ids, n_tokens, out, token=0, err=None, stream=None):
    check(lib.mlk_gather_f32(_p(table), vocab, dim, _p(ids), token, n_tokens, _p(out), _p(err),
                             _sp(stream)), "mlk_gather_f32")


def gather_quant(qtype, blocks, vocab, dim, ids, n_tokens, out, token=0, err=None, stream=None):
    check(lib.mlk_gather_quant(QUANT[qtype], _p(blocks), vocab, dim, _p(ids), token, n_tokens,
                               _p(out), _p(err), _sp(stream)), "mlk_gather_quant")


def quantize(qtype, x, rows, cols, blocks, stream=None):
    check(lib.mlk_quantize(QUANT[qtype], _p(x), rows, cols, _p(blocks), _sp(stream)),
          "mlk_quantize")


def linear_workspace_bytes(rows, in_features, out_features):
    """Bytes of the optional split-K workspace of a linear call (0: none used)."""
    return int(lib.mlk_linear_workspace_bytes(rows, in_features, out_features))


_linear_ws = {}  # device id -> DeviceBuffer grown to the largest request


def _workspace(workspace, rows, in_features, out_features):
    """(pointer, bytes) for a linear call: workspace is None (no split), a
    DeviceBuffer, or "auto" (a per-device buffer kept by this module and grown
    when a call needs more; growing frees the old one, which waits for the
    device, so do not use "auto" under graph capture)."""
    if workspace is None:
        return None, 0
    if isinstance(workspace, str):
        if workspace != "auto":
            raise ValueError(f"workspace must be None, a DeviceBuffer or 'auto', not {workspace!r}")
        need = linear_workspace_bytes(rows, in_features, out_features)
        if need == 0:
            return None, 0
        dev = C.c_int()
        check(lib.mlk_get_device(C.byref(dev)))
        buf = _linear_ws.get(dev.value)
        if buf is None or buf.nbytes < need:
            if buf is not None:
                buf.close()
            buf = _linear_ws[dev.value] = DeviceBuffer(need, np.uint8)
        return buf.ptr, buf.nbytes
    return _p(workspace), workspace.nbytes


def linear_quant(qtype, x, w_blocks, y, rows, in_features, out_features, bias=None,
                 stream=None, workspace="auto"):
    """y[rows, out] = x[rows, in] @ dequant(W)^T (+ bias)."""
    ws, ws_bytes = _workspace(workspace, rows, in_features, out_features)
    check(lib.mlk_linear_quant(QUANT[qtype], _p(x), _p(w_blocks), _p(bias), _p(y), rows,
                               in_features, out_features, ws, ws_bytes, _sp(stream)),
          "mlk_linear_quant")


def quant_planar_bytes(qtype, rows, cols):
    """Bytes of the planar layout of a [rows, cols] Q8_0 / Q4_0 matrix (0: none)."""
    return int(lib.mlk_quant_planar_bytes(QUANT[qtype], rows, cols))


def quant_to_planar(qtype, w_blocks, rows, cols, planar, stream=None):
    """Repack [rows, cols] blocks into the planar layout (a buffer of
    quant_planar_bytes bytes)."""
    check(lib.mlk_quant_to_planar(QUANT[qtype], _p(w_blocks), rows, cols, _p(planar),
                                  _sp(stream)), "mlk_quant_to_planar")


def linear_planar_workspace_bytes(rows, in_features, out_features):
    """Bytes of the workspace of linear_planar (required up to 32 rows)."""
    return int(lib.mlk_linear_planar_workspace_bytes(rows, in_features, out_features))


_planar_ws = {}  # device id -> DeviceBuffer grown to the largest request


def linear_planar(qtype, x, w_planar, y, rows, in_features, out_features, bias=None,
                  stream=None, workspace="auto"):
    """y[rows, out] = x[rows, in] @ dequant(W)^T (+ bias), W in the planar
    layout; workspace: a DeviceBuffer, or "auto" (a per-device buffer kept by
    this module, grown as needed)."""
    if isinstance(workspace, str):
        if workspace != "auto":
            raise ValueError(f"workspace must be a DeviceBuffer or 'auto', not {workspace!r}")
        need = max(linear_planar_workspace_bytes(rows, in_features, out_features), 16)
        dev = C.c_int()
        check(lib.mlk_get_device(C.byref(dev)))
        buf = _planar_ws.get(dev.value)
        if buf is None or buf.nbytes < need:
            if buf is not None:
                buf.close()
            buf = _planar_ws[dev.value] = DeviceBuffer(need, np.uint8)
        ws, ws_bytes = buf.ptr, buf.nbytes
    elif workspace is None:
        ws, ws_bytes = None, 0
    else:
        ws, ws_bytes = _p(workspace), workspace.nbytes
    check(lib.mlk_linear_planar(QUANT[qtype], _p(x), _p(w_planar), _p(bias), _p(y), rows,
                                in_features, out_features, ws, ws_bytes, _sp(stream)),
          "mlk_linear_planar")


def linear_f32(x, w, y, rows, in_features, out_features, bias=None, stream=None,
               workspace="auto"):
    """y[rows, out] = x[rows, in] @ W[out, in]^T (+ bias)."""
    ws, ws_bytes = _workspace(workspace, rows, in_features, out_features)
    check(lib.mlk_linear_f32(_p(x), _p(w), _p(bias), _p(y), rows, in_features, out_features,
                             ws, ws_bytes, _sp(stream)), "mlk_linear_f32")


def matmul(a, b, c, m, k, n, stream=None):
    """c[m, n] = a[m, k] @ b[k, n]."""
    check(lib.mlk_matmul_f32(_p(a), _p(b), _p(c), m, k, n, _sp(stream)), "mlk_matmul_f32")


def kv_write(k_cache, v_cache, n_layers, max_seq, n_kv_heads, head_dim, layer, k, v, n_tokens,
             positions=None, pos0=0, k_row_stride=None, v_row_stride=None, err=None,
             stream=None):
    """Copies k, v rows [n_tokens, n_kv_heads * head_dim] into cache slots
    (layer, positions[t] or pos0 + t) of caches [n_layers, max_seq,
    n_kv_heads, head_dim]."""
    row = n_kv_heads * head_dim
    check(lib.mlk_kv_write_f32(_p(k_cache), _p(v_cache), n_layers, max_seq, n_kv_heads, head_dim,
                               layer, _p(k), k_row_stride or row, _p(v), v_row_stride or row,
                               _p(positions), pos0, n_tokens, _p(err), _sp(stream)),
          "mlk_kv_write_f32")


def attention_workspace_bytes(n_tokens, n_heads, n_kv_heads, head_dim, max_ctx):
    return int(lib.mlk_attention_workspace_bytes(n_tokens, n_heads, n_kv_heads, head_dim,
                                                 max_ctx))


def attention_decode(q, k_cache, v_cache, n_layers, max_seq, n_heads, n_kv_heads, head_dim,
                     layer, n_tokens, out, max_ctx, positions=None, pos0=0, workspace=None,
                     workspace_bytes=0, q_row_stride=None, err=None, stream=None):
    """out [n_tokens, n_heads, head_dim] = attention of q rows over cache
    positions 0..pos of `layer` (pos = positions[t] or pos0 + t < max_ctx)."""
    check(lib.mlk_attention_decode_f32(_p(q), q_row_stride or n_heads * head_dim, _p(k_cache),
                                       _p(v_cache), n_layers, max_seq, n_heads, n_kv_heads,
                                       head_dim, layer, _p(positions), pos0, n_tokens, max_ctx,
                                       _p(out), _p(workspace), workspace_bytes, _p(err),
                                       _sp(stream)),
          "mlk_attention_decode_f32")


def attention_decode_noalloc(q, k_cache, v_cache, n_layers, max_seq, n_heads, n_kv_heads,
                             head_dim, layer, n_tokens, out, max_ctx, positions=None, pos0=0,
                             q_row_stride=None, err=None, stream=None):
    """attention_decode without a workspace: the chunk partials go to the
    library's fixed per-GPU scratch (attention_noalloc_scratch_bytes())."""
    check(lib.mlk_attention_decode_f32_noalloc(
        _p(q), q_row_stride or n_heads * head_dim, _p(k_cache), _p(v_cache), n_layers, max_seq,
        n_heads, n_kv_heads, head_dim, layer, _p(positions), pos0, n_tokens, max_ctx, _p(out),
        _p(err), _sp(stream)), "mlk_attention_decode_f32_noalloc")


def attention_noalloc_scratch_bytes():
    return int(lib.mlk_attention_noalloc_scratch_bytes())


def attention_prefill(q, k_cache, v_cache, n_layers, max_seq, n_heads, n_kv_heads, head_dim,
                      layer, pos0, n_tokens, out, q_row_stride=None, stream=None):
    """out [n_tokens, n_heads, head_dim]: token t (position pos0 + t) attends to
    cache positions 0..pos0 + t of `layer` (causal prompt chunk)."""
    check(lib.mlk_attention_prefill_f32(_p(q), q_row_stride or n_heads * head_dim, _p(k_cache),
                                        _p(v_cache), n_layers, max_seq, n_heads, n_kv_heads,
                                        head_dim, layer, pos0, n_tokens, _p(out), _sp(stream)),
          "mlk_attention_prefill_f32")


def quant_bytes(qtype, rows, cols):
    return int(lib.mlk_quant_bytes(QUANT[qtype], rows, cols))


def fill_normal(x, n, mean=0.0, std=1.0, seed=0, stream=None):
    check(lib.mlk_fill_normal_f32(_p(x), n, mean, std, seed, _sp(stream)), "mlk_fill_normal_f32")
