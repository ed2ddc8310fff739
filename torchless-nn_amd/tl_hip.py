"""ctypes binding of libtl (the C-ABI HIP library) and the device array type.

Under XP_RUNTIME=MI355X this module *is* the `xp` array namespace that the reference's
layers import from `backend` (reference backend.py:3-22). It offers the small CuPy-like
surface the forward path needs -- `array`, `zeros`, `empty`, `argmax`, `asnumpy`, dtypes and
a seeded `random.default_rng` -- over `DeviceTensor`, a pointer + shape + dtype + row pitch
that lives in HBM. There is no host fallback: if libtl.so is missing or no gfx950 device is
present, the first use raises.
"""
from __future__ import annotations

import ctypes
import math
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("TL_LIBRARY", os.path.join(_HERE, "libtl.so"))

# ---- enums (include/libtl.h) ----------------------------------------------------------
TL_OK, TL_ERR_INVALID, TL_ERR_HIP, TL_ERR_OOM, TL_ERR_NO_DEVICE, TL_ERR_BAD_INPUT, TL_ERR_UNSUPPORTED = range(7)
TL_ACT_NONE, TL_ACT_GELU, TL_ACT_SILU = 0, 1, 2
TL_B_NK, TL_B_KN = 0, 1
TL_EPI_STORE, TL_EPI_QKV_SPLIT, TL_EPI_GEGLU = 0, 1, 2
GEMM_TILES = {"auto": 0, "256x256": 1, "256x128": 2, "128x128": 3, "128x64": 4, "64x64": 5,
              "256x256w4": 6, "256x128w8": 7, "dma128x128": 8, "dma256x128w8": 9,
              "dma128x64s3": 10, "dma128x128s3": 11, "persist256x128w8": 12,
              "persist128x128": 13, "skinny": 14, "dma256x256w8": 15,
              "dma128x96": 16, "dma256x96w8": 17, "persist256x96w8": 18,
              "persist256x256w8": 19, "dma256x192w8": 20}
KFAMILY = {
    "gemm_mfma": 0, "gemm_batched": 1, "gemm_simt": 2, "layernorm": 3, "rmsnorm": 4,
    "softmax": 5, "rope": 6, "act": 7, "embed": 8, "argmax": 9, "attention": 10, "misc": 11,
}


class TLError(RuntimeError):
    """A libtl call failed; `.status` holds the tl_status code."""

    def __init__(self, status, message):
        super().__init__(f"libtl error {status}: {message}")
        self.status = status


class NoDeviceError(TLError):
    pass


class BadInputError(TLError, IndexError):
    """A kernel saw invalid data, e.g. a token id outside [0, vocab) (NumPy raises
    IndexError for the same input at reference transformer_adapters.py:150)."""


# ---- dtypes ---------------------------------------------------------------------------
class DType:
    __slots__ = ("name", "code", "itemsize", "host")

    def __init__(self, name, code, itemsize, host):
        self.name, self.code, self.itemsize, self.host = name, code, itemsize, np.dtype(host)

    def __repr__(self):
        return f"tl.{self.name}"

    @property
    def is_float(self):
        return self.code in (0, 1)


float32 = DType("float32", 0, 4, np.float32)
bfloat16 = DType("bfloat16", 1, 2, np.uint16)  # host view of bf16 is its raw uint16 bits
int32 = DType("int32", 2, 4, np.int32)
int64 = DType("int64", 3, 8, np.int64)
uint8 = DType("uint8", 4, 1, np.uint8)
pi = math.pi
_BY_NAME = {"float32": float32, "fp32": float32, "f32": float32, "bfloat16": bfloat16,
            "bf16": bfloat16, "int32": int32, "int64": int64, "uint8": uint8}


def as_dtype(dt) -> DType:
    if isinstance(dt, DType):
        return dt
    if isinstance(dt, str):
        return _BY_NAME[dt]
    nd = np.dtype(dt)
    if nd == np.float32 or nd == np.float64 or nd == np.float16:
        return float32
    if nd == np.uint8:
        return uint8
    if nd == np.int64 or nd == np.uint64 or nd == np.uint32:
        return int64
    if nd.kind in "iu":
        return int32
    if nd == np.bool_:
        return uint8
    raise TypeError(f"unsupported dtype {dt!r}")


# ---- bf16 host conversion (round to nearest even, as the gfx950 converter) ------------
def f32_to_bf16_bits(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + (0x7FFF + ((u >> 16) & 1))) >> 16).astype(np.uint16)
    if nan.any():
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


# ---- library loading ------------------------------------------------------------------
class _GemmDesc(ctypes.Structure):
    _fields_ = [
        ("M", ctypes.c_int64), ("N", ctypes.c_int64), ("K", ctypes.c_int64),
        ("A", ctypes.c_void_p), ("lda", ctypes.c_int64),
        ("B", ctypes.c_void_p), ("ldb", ctypes.c_int64), ("b_layout", ctypes.c_int32),
        ("C", ctypes.c_void_p), ("ldc", ctypes.c_int64),
        ("dtype_in", ctypes.c_int32), ("dtype_out", ctypes.c_int32),
        ("batch", ctypes.c_int64), ("batch_inner", ctypes.c_int64),
        ("sa_o", ctypes.c_int64), ("sa_i", ctypes.c_int64), ("sb_o", ctypes.c_int64),
        ("sb_i", ctypes.c_int64), ("sc_o", ctypes.c_int64), ("sc_i", ctypes.c_int64),
        ("bias", ctypes.c_void_p), ("residual", ctypes.c_void_p), ("ldr", ctypes.c_int64),
        ("sr_o", ctypes.c_int64), ("sr_i", ctypes.c_int64),
        ("act", ctypes.c_int32), ("divisor", ctypes.c_float), ("epilogue", ctypes.c_int32),
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("vt", ctypes.c_void_p),
        ("seq_len", ctypes.c_int64), ("n_heads_q", ctypes.c_int64),
        ("n_heads_kv", ctypes.c_int64), ("head_dim", ctypes.c_int64),
        ("kv_len", ctypes.c_int64), ("kv_pos0", ctypes.c_int64),
        ("family", ctypes.c_int32), ("tile", ctypes.c_int32),
        ("kv_pos0_dev", ctypes.c_void_p),
        ("norm_rows", ctypes.c_int32), ("norm_eps", ctypes.c_float),
    ]


_P, _I32, _I64, _F32, _F64, _SZ = (ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64,
                                   ctypes.c_float, ctypes.c_double, ctypes.c_size_t)
# name -> argtypes; every function returns int (tl_status) unless listed in _RESTYPES.
SIGNATURES = {
    "tl_version": [],
    "tl_last_error": [],
    "tl_device_count": [ctypes.POINTER(ctypes.c_int)],
    "tl_init": [ctypes.c_int, ctypes.POINTER(_P)],
    "tl_destroy": [_P],
    "tl_malloc": [_P, _SZ, ctypes.POINTER(_P)],
    "tl_free": [_P, _P],
    "tl_empty_cache": [_P],
    "tl_mem_stats": [_P, ctypes.POINTER(_SZ), ctypes.POINTER(_SZ)],
    "tl_workspace_bytes": [_P, ctypes.POINTER(_SZ)],
    "tl_memcpy_h2d": [_P, _P, _P, _SZ],
    "tl_memcpy_d2h": [_P, _P, _P, _SZ],
    "tl_memcpy_d2d": [_P, _P, _P, _SZ],
    "tl_memcpy2d_h2d": [_P, _P, _SZ, _P, _SZ, _SZ, _SZ],
    "tl_memcpy2d_d2h": [_P, _P, _SZ, _P, _SZ, _SZ, _SZ],
    "tl_memcpy2d_d2d": [_P, _P, _SZ, _P, _SZ, _SZ, _SZ],
    "tl_sync": [_P],
    "tl_prefetch_hint": [_P, _P, _I64],
    "tl_event_create": [_P, ctypes.POINTER(_P)],
    "tl_event_record": [_P, _P],
    "tl_event_elapsed_ms": [_P, _P, ctypes.POINTER(_F32)],
    "tl_event_destroy": [_P],
    "tl_kprof_enable": [_P, ctypes.c_uint32],
    "tl_kprof_reset": [_P],
    "tl_kprof_query": [_P, ctypes.c_int, ctypes.POINTER(_I64), ctypes.POINTER(_F64),
                       ctypes.POINTER(_F64), ctypes.POINTER(_F64)],
    "tl_fill": [_P, _P, _I64, _I32, _F64],
    "tl_cast": [_P, _P, _P, _I64, _I32, _I32],
    "tl_random_normal": [_P, _P, _I64, ctypes.c_uint64, ctypes.c_uint64, _F32, _F32, _I32],
    "tl_sample": [_P, _P, _I64, _I32, _I64, ctypes.c_uint64, ctypes.c_uint64, _P],
    "tl_take": [_P, _P, _I64, _I32, _P, _I64, _P],
    "tl_transpose2d": [_P, _P, _P, _I64, _I64, _I64, _I64, _I32],
    "tl_add": [_P, _P, _P, _P, _I64, _I32],
    "tl_transpose2d_gain": [_P, _P, _P, _I64, _I64, _I64, _I64, _P, _F32, _I32],
    "tl_patchify": [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _I32],
    "tl_vit_project": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I32],
    "tl_embed_fwd": [_P, _P, _I32, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _F32, _I32],
    "tl_layernorm_fwd": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _F32, _I32],
    "tl_rmsnorm_fwd": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _F32, _F32, _I32],
    "tl_softmax_fwd": [_P, _P, _P, _I64, _I64, _I64, _I64, _F32, _I32, _I64, _I64, _I32],
    "tl_rope_table": [_P, _P, _I64, _I64, _F64, _I64],
    "tl_rope_fwd": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I32],
    "tl_rope2_fwd": [_P, _P, _P, _I64, _I64, _P, _P, _I64, _I64, _P, _I64, _I64, _I32],
    "tl_act_fwd": [_P, _P, _P, _I64, _I32, _I32],
    "tl_argmax": [_P, _P, _I64, _I64, _I64, _I32, _P],
    "tl_gemm": [_P, ctypes.POINTER(_GemmDesc)],
    "tl_attention_fwd": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
                         _F32, _I32, _I64, _I32],
    "tl_attention_fwd_noalloc": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
                                 _I64, _F32, _I32, _I64, _I32],
    "tl_attention_decode_dev": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _F32,
                                _I64, _P, _P, _I32],
    "tl_graph_begin": [_P],
    "tl_graph_end": [_P, ctypes.POINTER(_P)],
    "tl_graph_launch": [_P, _P],
    "tl_graph_destroy": [_P, _P],
    "tl_rope_table_dev": [_P, _P, _I64, _I64, _F64, _P],
    "tl_rope2_dev": [_P, _P, _I64, _I64, _P, _I64, _I64, _I64, _P, _I64, _I64, _P, _I32],
    "tl_i64_add": [_P, _P, _I64],
    "tl_ids_append": [_P, _P, _P, _I64, _I64, _I64, _P, _I64],
}
_RESTYPES = {"tl_last_error": ctypes.c_char_p}

_lib = None


def load_library(path: str = LIB_PATH):
    """Load libtl.so and declare every exported signature. Raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(f"libtl.so not found at {path}: build it first "
                          f"(python -c 'import __graft_entry__ as g; g.build()')")
    lib = ctypes.CDLL(path)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPES.get(name, ctypes.c_int)
    _lib = lib
    return lib


def last_error() -> str:
    return load_library().tl_last_error().decode(errors="replace")


def check(rc: int, what: str = ""):
    if rc == TL_OK:
        return
    msg = last_error() or what
    if rc == TL_ERR_NO_DEVICE:
        raise NoDeviceError(rc, msg)
    if rc == TL_ERR_BAD_INPUT:
        raise BadInputError(rc, msg)
    if rc == TL_ERR_INVALID:
        raise TLError(rc, "invalid argument: " + msg)
    raise TLError(rc, msg)


def device_count() -> int:
    n = ctypes.c_int(0)
    check(load_library().tl_device_count(ctypes.byref(n)))
    return n.value


class Context:
    """One tl_ctx: a device and its in-order stream."""

    def __init__(self, device: int = 0):
        lib = load_library()
        h = ctypes.c_void_p()
        check(lib.tl_init(int(device), ctypes.byref(h)))
        self.handle = h
        self.device = device
        self.lib = lib

    def sync(self):
        check(self.lib.tl_sync(self.handle))

    def mem_stats(self):
        a, b = ctypes.c_size_t(), ctypes.c_size_t()
        check(self.lib.tl_mem_stats(self.handle, ctypes.byref(a), ctypes.byref(b)))
        return a.value, b.value

    def empty_cache(self):
        check(self.lib.tl_empty_cache(self.handle))

    def workspace_bytes(self):
        n = ctypes.c_size_t()
        check(self.lib.tl_workspace_bytes(self.handle, ctypes.byref(n)))
        return n.value

    def destroy(self):
        if self.handle:
            check(self.lib.tl_destroy(self.handle))
            self.handle = None


_ctx = None


def ctx() -> Context:
    global _ctx
    if _ctx is None:
        _ctx = Context(int(os.environ.get("TL_DEVICE", "0")))
    return _ctx


def lib():
    return ctx().lib


def synchronize():
    ctx().sync()


# ---- device memory --------------------------------------------------------------------
class DeviceBuffer:
    """One tl_malloc allocation. `version` counts the writes made into it through this
    module (by any view of it), so data derived from its contents can tell it is stale."""
    __slots__ = ("ptr", "nbytes", "_ctx", "version", "__weakref__")

    def __init__(self, nbytes: int):
        c = ctx()
        p = ctypes.c_void_p()
        check(c.lib.tl_malloc(c.handle, int(nbytes), ctypes.byref(p)))
        self.ptr, self.nbytes, self._ctx, self.version = p.value, int(nbytes), c, 0

    def __del__(self):
        try:
            if self.ptr:
                self._ctx.lib.tl_free(self._ctx.handle, self.ptr)
                self.ptr = None
        except Exception:
            pass


def _prod(shape):
    n = 1
    for s in shape:
        n *= int(s)
    return n


def _norm_shape(shape):
    if isinstance(shape, (int, np.integer)):
        return (int(shape),)
    return tuple(int(s) for s in shape)


class DeviceTensor:
    """An array in HBM: shape, dtype and the pitch (in elements) between consecutive
    rows of the last dimension. Rows are padded only where a kernel benefits (e.g. the
    50257-wide logits use a pitch that keeps every row 16-byte aligned)."""

    __slots__ = ("shape", "dtype", "pitch", "buf", "offset", "_aux", "__weakref__")

    def __init__(self, shape, dtype, pitch=None, buf=None, offset=0):
        self.shape = _norm_shape(shape)
        self.dtype = as_dtype(dtype)
        cols = self.shape[-1] if self.shape else 1
        self.pitch = int(pitch) if pitch is not None else cols
        if self.pitch < cols:
            raise ValueError("pitch smaller than the last dimension")
        if buf is None:
            buf = DeviceBuffer(max(1, self.nrows * self.pitch * self.dtype.itemsize))
        elif self.size:
            # a view must lie inside its buffer: kernels take raw pointers and cannot check
            end = int(offset) + ((self.nrows - 1) * self.pitch + cols) * self.dtype.itemsize
            if int(offset) < 0 or end > buf.nbytes:
                raise ValueError(f"view of {end - int(offset)} bytes at offset {int(offset)} "
                                 f"exceeds its {buf.nbytes}-byte buffer")
        self.buf, self.offset = buf, int(offset)
        self._aux = None  # device-side derived data (e.g. a packed weight), by _version

    @property
    def _version(self) -> int:
        """Write count of the underlying buffer: it changes whenever any view of the buffer
        is written through this module (set, fill, or a kernel's out= / C= operand)."""
        return self.buf.version

    @_version.setter
    def _version(self, value):
        self.buf.version = int(value)

    # -- geometry
    @property
    def ptr(self) -> int:
        return self.buf.ptr + self.offset

    @property
    def ndim(self):
        return len(self.shape)

    @property
    def size(self):
        return _prod(self.shape)

    @property
    def ncols(self):
        return self.shape[-1] if self.shape else 1

    @property
    def nrows(self):
        return _prod(self.shape[:-1]) if self.shape else 1

    @property
    def nbytes(self):
        return self.size * self.dtype.itemsize

    @property
    def contiguous(self):
        return self.pitch == self.ncols

    def __len__(self):
        if not self.shape:
            raise TypeError("len() of a 0-d tensor")
        return self.shape[0]

    def __getitem__(self, key):
        """Basic indexing (integers, negative ones included, and step-1 slices) as a view of
        the same memory, where the result keeps one row pitch: evenly spaced whole rows with
        a column range (e.g. the notebook's `tokens[:, a:]`, `probs[0, -1]`), or one element.
        Other selections raise NotImplementedError rather than copy."""
        if not isinstance(key, tuple):
            key = (key,)
        if any(k is Ellipsis or k is None for k in key):
            raise NotImplementedError("indexing with ... or None")
        if not self.shape or len(key) > self.ndim:
            raise IndexError(f"too many indices for a {self.ndim}-d tensor")
        key = key + (slice(None),) * (self.ndim - len(key))
        lead, last = key[:-1], key[-1]
        rows = np.arange(self.nrows).reshape(self.shape[:-1])[lead]  # numpy checks the bounds
        row_shape, flat = rows.shape, rows.reshape(-1)
        n = self.ncols
        if isinstance(last, slice):
            c0, c1, step = last.indices(n)
            if step != 1:
                raise NotImplementedError("slices with a step")
            ncol, col_shape = max(0, c1 - c0), (max(0, c1 - c0),)
        else:
            c0 = int(last) + (n if int(last) < 0 else 0)
            if not 0 <= c0 < n:
                raise IndexError(f"index {int(last)} out of range for size {n}")
            ncol, col_shape = 1, ()
        if flat.size == 0 or ncol == 0:
            return DeviceTensor(row_shape + col_shape, self.dtype, buf=self.buf, offset=self.offset)
        off = self.offset + (int(flat[0]) * self.pitch + c0) * self.dtype.itemsize
        if flat.size == 1:
            return DeviceTensor(row_shape + col_shape, self.dtype, buf=self.buf, offset=off)
        steps = np.diff(flat)
        if col_shape == () or not np.all(steps == steps[0]):
            raise NotImplementedError("this selection is not a view with one row pitch")
        return DeviceTensor(row_shape + col_shape, self.dtype, pitch=int(steps[0]) * self.pitch,
                            buf=self.buf, offset=off)

    def __repr__(self):
        return f"DeviceTensor(shape={self.shape}, dtype={self.dtype}, pitch={self.pitch})"

    # -- host transfer
    def get_raw(self) -> np.ndarray:
        """Copy to host without conversion (bf16 comes back as uint16 bits)."""
        c = ctx()
        host = np.empty((self.nrows, self.ncols), dtype=self.dtype.host)
        if self.size:
            es = self.dtype.itemsize
            check(c.lib.tl_memcpy2d_d2h(c.handle, host.ctypes.data, self.ncols * es, self.ptr,
                                        self.pitch * es, self.ncols * es, self.nrows))
        return host.reshape(self.shape)

    def get(self) -> np.ndarray:
        """Copy to host (CuPy's `.get()`); bf16 is widened to float32."""
        raw = self.get_raw()
        return bf16_bits_to_f32(raw).reshape(self.shape) if self.dtype is bfloat16 else raw

    def set(self, host):
        """Upload a host array of the same shape (converted to this tensor's dtype)."""
        host = np.asarray(host)
        if host.shape != self.shape:
            raise ValueError(f"shape mismatch: {host.shape} vs {self.shape}")
        raw = _to_host_raw(host, self.dtype).reshape(self.nrows, self.ncols)
        c = ctx()
        if self.size:
            es = self.dtype.itemsize
            check(c.lib.tl_memcpy2d_h2d(c.handle, self.ptr, self.pitch * es, raw.ctypes.data,
                                        self.ncols * es, self.ncols * es, self.nrows))
        self._version += 1
        return self

    # -- views and small device ops
    def reshape(self, *shape):
        if len(shape) == 1 and not isinstance(shape[0], (int, np.integer)):
            shape = tuple(shape[0])
        shape = list(int(s) for s in shape)
        if -1 in shape:
            i = shape.index(-1)
            rest = _prod(shape[:i] + shape[i + 1:])
            shape[i] = self.size // rest if rest else 0
        shape = tuple(shape)
        if _prod(shape) != self.size:
            raise ValueError(f"cannot reshape {self.shape} into {shape}")
        if shape and self.shape and shape[-1] == self.ncols:
            return DeviceTensor(shape, self.dtype, self.pitch, self.buf, self.offset)
        if not self.contiguous:
            raise ValueError("reshape of a padded tensor must keep the last dimension")
        return DeviceTensor(shape, self.dtype, None, self.buf, self.offset)

    def fill(self, value):
        if not self.contiguous:
            raise ValueError("fill of a padded tensor")
        c = ctx()
        check(c.lib.tl_fill(c.handle, self.ptr, self.size, self.dtype.code, float(value)))
        self._version += 1
        return self

    def astype(self, dtype, copy=True):
        dtype = as_dtype(dtype)
        if dtype is self.dtype and not copy:
            return self
        if not self.contiguous:
            raise ValueError("astype of a padded tensor")
        out = DeviceTensor(self.shape, dtype)
        c = ctx()
        if dtype is self.dtype:
            check(c.lib.tl_memcpy_d2d(c.handle, out.ptr, self.ptr, self.nbytes))
        else:
            check(c.lib.tl_cast(c.handle, self.ptr, out.ptr, self.size, self.dtype.code, dtype.code))
        return out

    def copy(self):
        return self.astype(self.dtype, copy=True)

    def __add__(self, other):
        if not isinstance(other, DeviceTensor) or other.shape != self.shape or other.dtype is not self.dtype:
            raise TypeError("DeviceTensor + needs a DeviceTensor of the same shape and dtype")
        if not (self.contiguous and other.contiguous):
            raise ValueError("add of padded tensors")
        out = DeviceTensor(self.shape, self.dtype)
        c = ctx()
        check(c.lib.tl_add(c.handle, self.ptr, other.ptr, out.ptr, self.size, self.dtype.code))
        return out


def _wrote(*tensors):
    """Record a write into each given tensor's buffer (None entries are skipped)."""
    for t in tensors:
        if t is not None:
            t.buf.version += 1


def _to_host_raw(host: np.ndarray, dtype: DType) -> np.ndarray:
    if dtype is bfloat16:
        return f32_to_bf16_bits(np.asarray(host, dtype=np.float32))
    return np.ascontiguousarray(host, dtype=dtype.host)


# ---- namespace functions (the `xp` surface) --------------------------------------------
def empty(shape, dtype=float32, pitch=None) -> DeviceTensor:
    return DeviceTensor(shape, dtype, pitch)


def zeros(shape, dtype=float32) -> DeviceTensor:
    return DeviceTensor(shape, dtype).fill(0)


def array(obj, dtype=None) -> DeviceTensor:
    """Upload (CuPy's `xp.array`). Float data defaults to the backend FLOAT_TYPE."""
    if isinstance(obj, DeviceTensor):
        return obj.astype(dtype if dtype is not None else obj.dtype)
    host = np.asarray(obj)
    if dtype is None:
        if host.dtype.kind == "f":
            import backend  # the active FLOAT_TYPE
            dtype = backend.FLOAT_TYPE
        else:
            dtype = as_dtype(host.dtype)
    dtype = as_dtype(dtype)
    return DeviceTensor(host.shape, dtype).set(host)


asarray = array


def arange(start, stop=None, step=1, dtype=None) -> DeviceTensor:
    """xp.arange (reference demo.ipynb:1531 samples from xp.arange(0, vocab_size))."""
    host = np.arange(start, stop, step) if stop is not None else np.arange(start)
    if dtype is not None:
        host = host.astype(as_dtype(dtype).host if as_dtype(dtype) is not bfloat16 else np.float32)
    return array(host, dtype=dtype)


def copy_into(dst: DeviceTensor, src: DeviceTensor):
    """dst[...] = src for contiguous tensors of one shape and dtype (stream-ordered)."""
    if dst.shape != src.shape or dst.dtype is not src.dtype or not (dst.contiguous and src.contiguous):
        raise ValueError("copy_into needs contiguous tensors of one shape and dtype")
    c = ctx()
    check(c.lib.tl_memcpy_d2d(c.handle, dst.ptr, src.ptr, src.nbytes))
    _wrote(dst)
    return dst


def concatenate(tensors, axis=0) -> DeviceTensor:
    """xp.concatenate of same-dtype tensors that agree except along `axis` (reference
    demo.ipynb:1533 appends each sampled token with axis=1), as device row copies."""
    tensors = list(tensors)
    if not tensors:
        raise ValueError("need at least one tensor to concatenate")
    first = tensors[0]
    nd = first.ndim
    axis = axis + nd if axis < 0 else axis
    if nd == 0 or not 0 <= axis < nd:
        raise ValueError(f"axis {axis} out of range for {nd}-d tensors")
    for t in tensors:
        if t.dtype is not first.dtype or t.ndim != nd or any(
                t.shape[i] != first.shape[i] for i in range(nd) if i != axis):
            raise ValueError("concatenate needs one dtype and matching shapes off the axis")
    shape = list(first.shape)
    shape[axis] = sum(t.shape[axis] for t in tensors)
    out = DeviceTensor(tuple(shape), first.dtype)
    es = first.dtype.itemsize
    c = ctx()
    outer = _prod(shape[:axis])            # blocks along the leading axes
    at = 0                                 # element offset inside each block of `out`
    block = _prod(shape[axis:])            # elements of one block of `out`
    for t in tensors:
        inner = _prod(t.shape[axis:])      # elements of one block of t
        if t.size:
            if axis == nd - 1 or t.contiguous:
                if axis == nd - 1:         # each row of t is one block
                    check(c.lib.tl_memcpy2d_d2d(c.handle, out.ptr + at * es, block * es, t.ptr,
                                                t.pitch * es, inner * es, outer))
                else:
                    check(c.lib.tl_memcpy2d_d2d(c.handle, out.ptr + at * es, block * es, t.ptr,
                                                inner * es, inner * es, outer))
            else:
                raise NotImplementedError("concatenate of a padded tensor off its last axis")
        at += inner
    _wrote(out)
    return out


def asnumpy(t) -> np.ndarray:
    return t.get() if isinstance(t, DeviceTensor) else np.asarray(t)


def argmax(t: DeviceTensor, axis=-1, out=None) -> DeviceTensor:
    """First index of the maximum along the last axis, int64 (reference network.py:135, 158).
    `out`, if given, is a contiguous int64 tensor with one element per row."""
    if axis not in (-1, t.ndim - 1):
        raise NotImplementedError("argmax is implemented over the last axis")
    if out is None:
        out = DeviceTensor(t.shape[:-1] if t.ndim > 1 else (1,), int64)
    elif out.dtype is not int64 or out.size != t.nrows or not out.contiguous:
        raise ValueError("argmax out must be a contiguous int64 tensor, one element per row")
    c = ctx()
    check(c.lib.tl_argmax(c.handle, t.ptr, t.nrows, t.ncols, t.pitch, t.dtype.code, out.ptr))
    _wrote(out)
    return out


def random_normal(shape, seed, stream=0, mean=0.0, std=1.0, dtype=float32, out=None) -> DeviceTensor:
    """mean + std * N(0, 1) drawn on the device (Philox4x32-10 keyed by `seed`, counter
    stream `stream`, Box-Muller). Same (seed, stream) -> same values for any dtype/shape
    prefix. `out` (contiguous) is filled in place."""
    out = out if out is not None else DeviceTensor(shape, dtype)
    if not out.contiguous:
        raise ValueError("random_normal needs a contiguous tensor")
    c = ctx()
    check(c.lib.tl_random_normal(c.handle, out.ptr, out.size, int(seed) & (2 ** 64 - 1),
                                 int(stream) & (2 ** 64 - 1), float(mean), float(std),
                                 out.dtype.code))
    out._version += 1
    return out


class _Rng:
    """Seeded host generator whose draws land in HBM (reference backend.py:28 keeps an
    unseeded `default_rng`; parity runs pass a seed)."""

    def __init__(self, seed=None):
        self._g = np.random.default_rng(seed)

    def standard_normal(self, size, dtype=float32):
        return array(self._g.standard_normal(_norm_shape(size), dtype=np.float32), dtype=dtype)

    def random(self, size, dtype=float32):
        return array(self._g.random(_norm_shape(size), dtype=np.float32), dtype=dtype)

    def integers(self, low, high=None, size=None, dtype=int64):
        return array(self._g.integers(low, high, size=size), dtype=dtype)


# key and next counter stream of xp.random.choice (seeded from TL_SEED; xp.random.seed sets it)
_SAMPLER = {"seed": int(os.environ.get("TL_SEED", "0")), "stream": 0}


def _choice(a, size=None, replace=True, p=None):
    """xp.random.choice(a, size, p=probs) (reference demo.ipynb:1531): draws on the device
    from the categorical distribution p (tl_sample; each call takes the next Philox stream
    of the sampler's key), then gathers the drawn entries of `a` (an int means arange(a)).
    Returns a device tensor of shape `size` (a's dtype, int64 for an int `a`)."""
    if p is None or not replace:
        raise NotImplementedError("choice is implemented with p given and replace=True")
    if not isinstance(p, DeviceTensor):
        p = array(np.asarray(p, dtype=np.float32), dtype=float32)
    if p.ndim != 1 or not p.contiguous:
        raise ValueError("p must be one contiguous row of probabilities")
    n_cand = int(a) if not isinstance(a, DeviceTensor) else a.size
    if n_cand != p.size:
        raise ValueError(f"a has {n_cand} entries but p has {p.size}")
    shape = () if size is None else ((int(size),) if isinstance(size, (int, np.integer))
                                     else tuple(int(v) for v in size))
    n = _prod(shape)
    idx = DeviceTensor((max(n, 1),), int64)
    c = ctx()
    stream = _SAMPLER["stream"]
    _SAMPLER["stream"] += 1
    check(c.lib.tl_sample(c.handle, p.ptr, p.size, p.dtype.code, n, _SAMPLER["seed"] & (2 ** 64 - 1),
                          stream, idx.ptr))
    if not isinstance(a, DeviceTensor):
        return DeviceTensor(shape, int64, buf=idx.buf, offset=idx.offset)
    if a.ndim != 1 or not a.contiguous:
        raise ValueError("a must be a 1-d contiguous tensor or an int")
    out = DeviceTensor(shape, a.dtype)
    check(c.lib.tl_take(c.handle, a.ptr, a.size, a.dtype.itemsize, idx.ptr, n, out.ptr))
    return out


def _seed(seed=None):
    """xp.random.seed: fixes the sampler's key and restarts its streams."""
    _SAMPLER["seed"] = int(seed) if seed is not None else int(os.environ.get("TL_SEED", "0"))
    _SAMPLER["stream"] = 0


class random:  # noqa: N801  (mirrors `xp.random`)
    default_rng = _Rng
    choice = staticmethod(_choice)
    seed = staticmethod(_seed)


# ---- kernel wrappers used by the layers ------------------------------------------------
def _c():
    c = ctx()
    return c.lib, c.handle


def gemm(A: DeviceTensor, B: DeviceTensor, *, M, N, K, lda, ldb, b_layout, C=None, ldc=0,
         out_dtype=None, batch=1, batch_inner=1, sa=(0, 0), sb=(0, 0), sc=(0, 0), bias=None,
         residual=None, ldr=0, sr=(0, 0), act=TL_ACT_NONE, divisor=1.0, qkv=None,
         family="gemm_mfma", tile="auto", geglu=False, norm_eps=None):
    """One tl_gemm call. qkv = (q, k, vt, T, Hq, Hkv, D[, kv_len, kv_pos0]) selects the
    split epilogue; kv_pos0 may be a one-element int64 DeviceTensor (the cache position
    read on the device when the kernel runs). norm_eps (M <= 16) scales each row of the
    product by 1 / sqrt(mean(A_row^2) + norm_eps): RMSNorm(A) @ B when B carries the norm's
    gain."""
    pos_dev = None
    if qkv is not None:
        q, k, vt, T, Hq, Hkv, Dh = qkv[:7]
        kv_len, kv_pos0 = (qkv[7], qkv[8]) if len(qkv) > 7 else (0, 0)
        if isinstance(kv_pos0, DeviceTensor):
            pos_dev, kv_pos0 = _position_ptr(kv_pos0), 0
        epi, qp, kp, vp = TL_EPI_QKV_SPLIT, q.ptr, k.ptr, vt.ptr
    else:
        epi = TL_EPI_GEGLU if geglu else TL_EPI_STORE
        qp = kp = vp = None
        T = Hq = Hkv = Dh = kv_len = kv_pos0 = 0
    code_in = A.dtype.code
    # one positional constructor call, in the field order of _GemmDesc
    d = _GemmDesc(M, N, K, A.ptr, lda, B.ptr, ldb, b_layout,
                  C.ptr if C is not None else None, ldc, code_in,
                  as_dtype(out_dtype).code if out_dtype is not None else code_in,
                  batch, batch_inner, sa[0], sa[1], sb[0], sb[1], sc[0], sc[1],
                  bias.ptr if bias is not None else None,
                  residual.ptr if residual is not None else None, ldr, sr[0], sr[1],
                  act, float(divisor), epi, qp, kp, vp, T, Hq, Hkv, Dh, kv_len, kv_pos0,
                  KFAMILY[family], GEMM_TILES[tile], pos_dev, int(norm_eps is not None),
                  float(norm_eps) if norm_eps is not None else 0.0)
    lib_, h = _c()
    check(lib_.tl_gemm(h, ctypes.byref(d)))
    if qkv is not None:
        _wrote(qkv[0], qkv[1], qkv[2])
    else:
        _wrote(C)


def layernorm(x: DeviceTensor, gamma, beta, eps, out=None):
    out = out if out is not None else DeviceTensor(x.shape, x.dtype)
    lib_, h = _c()
    check(lib_.tl_layernorm_fwd(h, x.ptr, gamma.ptr, beta.ptr, out.ptr, x.nrows, x.ncols,
                                x.pitch, out.pitch, float(eps), x.dtype.code))
    _wrote(out)
    return out


def rmsnorm(x: DeviceTensor, gamma, eps, gamma_offset=0.0, out=None):
    out = out if out is not None else DeviceTensor(x.shape, x.dtype)
    lib_, h = _c()
    check(lib_.tl_rmsnorm_fwd(h, x.ptr, gamma.ptr, out.ptr, x.nrows, x.ncols, x.pitch,
                              out.pitch, float(eps), float(gamma_offset), x.dtype.code))
    _wrote(out)
    return out


def prefetch_hint(t: DeviceTensor):
    """Have the next layernorm / rmsnorm launch also read `t`'s memory (one word per 128-byte
    line) so a product right after the norm finds it in the device caches. Advisory: no
    result changes; up to 4 tensors per norm launch."""
    span = ((t.nrows - 1) * t.pitch + t.ncols) * t.dtype.itemsize if t.size else 0
    lib_, h = _c()
    check(lib_.tl_prefetch_hint(h, t.ptr, span))


def softmax(x: DeviceTensor, temperature=1.0, causal=False, period=1, offset=0, out=None):
    out = out if out is not None else DeviceTensor(x.shape, x.dtype, x.pitch)
    lib_, h = _c()
    check(lib_.tl_softmax_fwd(h, x.ptr, out.ptr, x.nrows, x.ncols, x.pitch, out.pitch,
                              float(temperature), int(bool(causal)), int(period), int(offset),
                              x.dtype.code))
    _wrote(out)
    return out


def rope_table(seq_len, head_dim, base=10000.0, pos0=0) -> DeviceTensor:
    t = DeviceTensor((2, seq_len, head_dim // 2), float32)
    lib_, h = _c()
    check(lib_.tl_rope_table(h, t.ptr, seq_len, head_dim, float(base), int(pos0)))
    return t


def rope(x: DeviceTensor, table: DeviceTensor, out=None, seq_len=None, n_seq=None,
         seq_stride=None):
    """Rotate-half RoPE over the last two dims [.., T, D] of a contiguous tensor, or over
    `n_seq` sequences of `seq_len` rows placed `seq_stride` elements apart (a cache slice;
    then x/out are the first row of the slice and the op may run in place)."""
    if not x.contiguous:
        raise ValueError("rope needs a contiguous tensor")
    D = x.shape[-1]
    T = seq_len if seq_len is not None else x.shape[-2]
    n = n_seq if n_seq is not None else x.size // (T * D)
    stride = seq_stride if seq_stride is not None else T * D
    out = out if out is not None else DeviceTensor(x.shape, x.dtype)
    if n > 0:
        span = ((n - 1) * stride + T * D) * x.dtype.itemsize
        for t in (x, out):
            if t.offset + span > t.buf.nbytes:
                raise ValueError(f"rope over {n} sequences {stride} elements apart runs past "
                                 f"the end of its buffer")
    lib_, h = _c()
    check(lib_.tl_rope_fwd(h, x.ptr, out.ptr, table.ptr, n, T, D, stride, x.dtype.code))
    _wrote(out)
    return out


def _rope_set(x: DeviceTensor, T, D, n_seq, seq_stride):
    """(n, stride) of one RoPE operand, checked against its buffer (in place)."""
    if not x.contiguous:
        raise ValueError("rope needs a contiguous tensor")
    if x.shape[-1] != D:
        raise ValueError("rope operands must share the head dim")
    n = n_seq if n_seq is not None else x.size // (T * D)
    stride = seq_stride if seq_stride is not None else T * D
    if n > 0 and x.offset + ((n - 1) * stride + T * D) * x.dtype.itemsize > x.buf.nbytes:
        raise ValueError(f"rope over {n} sequences {stride} elements apart runs past the end "
                         f"of its buffer")
    return n, stride


def rope2(x1: DeviceTensor, x2: DeviceTensor, table: DeviceTensor, seq_len, n_seq1=None,
          seq_stride1=None, n_seq2=None, seq_stride2=None):
    """In-place rotate-half RoPE of two tensors by the same `seq_len` positions in one launch
    (the queries and the new cache keys of an attention call); each operand is either packed
    [.., T, D] or `n_seq` sequences `seq_stride` elements apart, as in `rope`."""
    if x1.dtype is not x2.dtype:
        raise ValueError("rope2 operands must share a dtype")
    D, T = x1.shape[-1], seq_len
    n1, st1 = _rope_set(x1, T, D, n_seq1, seq_stride1)
    n2, st2 = _rope_set(x2, T, D, n_seq2, seq_stride2)
    lib_, h = _c()
    check(lib_.tl_rope2_fwd(h, x1.ptr, x1.ptr, n1, st1, x2.ptr, x2.ptr, n2, st2, table.ptr, T, D,
                            x1.dtype.code))
    _wrote(x1, x2)
    return x1, x2


def activation(x: DeviceTensor, act: int, out=None):
    if not x.contiguous:
        raise ValueError("activation needs a contiguous tensor")
    out = out if out is not None else DeviceTensor(x.shape, x.dtype)
    lib_, h = _c()
    check(lib_.tl_act_fwd(h, x.ptr, out.ptr, x.size, int(act), x.dtype.code))
    _wrote(out)
    return out


def embed(ids: DeviceTensor, table: DeviceTensor, pos, seq_len, pos0=0, out_shape=None,
          scale=1.0, out=None, ld_out=None):
    """out[t] = table[ids[t]] * scale (+ pos[pos0 + t % seq_len]). With `out`, row t is
    written at out + t * ld_out elements (e.g. one row per image of a token sequence)."""
    V, C = table.shape
    if out is None:
        out = DeviceTensor(out_shape or (ids.size, C), table.dtype)
        ld_out = out.pitch
    elif ids.size and out.offset + ((ids.size - 1) * ld_out + C) * out.dtype.itemsize > out.buf.nbytes:
        raise ValueError("embedding rows run past the end of the output buffer")
    lib_, h = _c()
    check(lib_.tl_embed_fwd(h, ids.ptr, ids.dtype.code, table.ptr,
                            pos.ptr if pos is not None else None, out.ptr, ids.size, seq_len,
                            pos0, V, C, ld_out, float(scale), table.dtype.code))
    _wrote(out)
    return out


def patchify(x: DeviceTensor, patch, dtype=None) -> DeviceTensor:
    """[B, C, H, W] -> [B, (H/p0)(W/p1), p0 p1 C] (reference transformer_adapters.py:39-47)."""
    if not x.contiguous or x.ndim != 4:
        raise ValueError("patchify needs a contiguous [B, C, H, W] tensor")
    B, C, H, W = x.shape
    p0, p1 = patch
    if H % p0 or W % p1:
        raise ValueError(f"image {H}x{W} is not a whole number of {p0}x{p1} patches")
    out = DeviceTensor((B, (H // p0) * (W // p1), p0 * p1 * C), dtype or x.dtype)
    lib_, h = _c()
    check(lib_.tl_patchify(h, x.ptr, out.ptr, B, C, H, W, p0, p1, x.dtype.code, out.dtype.code))
    return out


def vit_project_ok(x: DeviceTensor, patch, dim, n_cls_reg) -> bool:
    """Whether tl_vit_project takes this ViT front end (bf16, K = p0 p1 C <= 64 and a
    multiple of 8, at most 64 patches, dim a multiple of 96, n_cls_reg <= 64)."""
    if x.dtype is not bfloat16 or x.ndim != 4 or not x.contiguous:
        return False
    B, C, H, W = x.shape
    p0, p1 = patch
    K, L = p0 * p1 * C, (H // p0) * (W // p1)
    return (H % p0 == 0 and W % p1 == 0 and K <= 64 and K % 8 == 0 and L <= 64 and
            dim % 96 == 0 and dim <= 4096 and 0 <= n_cls_reg <= 64)


def vit_project(x: DeviceTensor, w: DeviceTensor, cls_reg: DeviceTensor, pos: DeviceTensor,
                patch, out: DeviceTensor):
    """The ViT front end in one launch (reference transformer_adapters.py:34-55): out [B, R + L,
    dim] = class/register tokens + positions, then patches(x) @ w^T + positions; w is the
    projection as [dim, K] (the packed form). See vit_project_ok for the shapes it takes."""
    B, C, H, W = x.shape
    R, dim = cls_reg.shape
    K, L = patch[0] * patch[1] * C, (H // patch[0]) * (W // patch[1])
    if (tuple(w.shape) != (dim, K) or tuple(pos.shape) != (R + L, dim) or
            tuple(out.shape) != (B, R + L, dim)):
        raise ValueError("vit_project: w [dim, K], pos [R + L, dim] and out [B, R + L, dim] expected")
    if not all(t.contiguous for t in (x, w, cls_reg, pos, out)):
        raise ValueError("vit_project needs contiguous tensors")
    lib_, h = _c()
    check(lib_.tl_vit_project(h, x.ptr, w.ptr, cls_reg.ptr, pos.ptr, out.ptr, B, C, H, W,
                              patch[0], patch[1], dim, R, x.dtype.code))
    _wrote(out)
    return out


def attention(q: DeviceTensor, k: DeviceTensor, vt: DeviceTensor, out: DeviceTensor, *,
              n_heads_q, n_heads_kv, divisor, causal=True, offset=0, seq_k=None):
    """Fused attention: q [B, Hq, Tq, D], k [B, Hkv, Lk, D], vt [B, Hkv, D, Lk] (the first
    `seq_k` keys valid, all Lk by default) -> out [B, Tq, Hq*D] (row pitch out.pitch).
    Raises TLError(TL_ERR_UNSUPPORTED) for shapes the kernel does not take."""
    B, Hq, Tq, D = q.shape
    Lk = k.shape[2]
    Tk = Lk if seq_k is None else seq_k
    lib_, h = _c()
    check(lib_.tl_attention_fwd(h, q.ptr, k.ptr, vt.ptr, out.ptr, B, n_heads_q, n_heads_kv, Tq,
                                Tk, D, out.pitch, int(offset), float(divisor), int(bool(causal)),
                                Lk, q.dtype.code))
    _wrote(out)
    return out


def _position_ptr(pos: DeviceTensor):
    if pos.dtype is not int64 or pos.size != 1:
        raise ValueError("a device position is a one-element int64 tensor")
    return pos.ptr


def attention_decode_dev(q: DeviceTensor, k: DeviceTensor, vt: DeviceTensor, out: DeviceTensor,
                         pos: DeviceTensor, *, n_heads_q, n_heads_kv, divisor, rope=None):
    """Causal decode attention at a device position: q [B, Hq, Tq, D] at positions
    *pos .. *pos + Tq - 1 over the cache k [B, Hkv, L, D] / vt [B, Hkv, D, L]. With `rope`
    (the float [2, Tq, D/2] table of those positions) q and the new cache keys come in
    unrotated; the kernel rotates both and writes the rotated keys back into k."""
    B, Hq, Tq, D = q.shape
    if rope is not None and (rope.dtype is not float32 or rope.shape != (2, Tq, D // 2)):
        raise ValueError("the RoPE table must be float32 [2, Tq, D/2]")
    lib_, h = _c()
    check(lib_.tl_attention_decode_dev(h, q.ptr, k.ptr, vt.ptr, out.ptr, B, n_heads_q,
                                       n_heads_kv, Tq, D, out.pitch, float(divisor), k.shape[2],
                                       _position_ptr(pos), rope.ptr if rope is not None else None,
                                       q.dtype.code))
    _wrote(out, k if rope is not None else None)
    return out


def rope_table_dev(table: DeviceTensor, pos: DeviceTensor, base=10000.0) -> DeviceTensor:
    """Fill `table` [2, T, D/2] (float32) with cos/sin of positions *pos .. *pos + T - 1."""
    _, T, half = table.shape
    lib_, h = _c()
    check(lib_.tl_rope_table_dev(h, table.ptr, T, 2 * half, float(base), _position_ptr(pos)))
    _wrote(table)
    return table


def rope2_dev(x1: DeviceTensor, cache: DeviceTensor, table: DeviceTensor, pos: DeviceTensor):
    """In place: rotate x1 [.., T, D] by the table's T positions, and the same T rows of
    every sequence of `cache` [.., L, D] starting at row *pos."""
    if x1.dtype is not cache.dtype or not (x1.contiguous and cache.contiguous):
        raise ValueError("rope2_dev needs contiguous operands of one dtype")
    T, D = x1.shape[-2], x1.shape[-1]
    L = cache.shape[-2]
    if cache.shape[-1] != D or table.shape[1] != T:
        raise ValueError("rope2_dev operands disagree on T or D")
    lib_, h = _c()
    check(lib_.tl_rope2_dev(h, x1.ptr, x1.size // (T * D), T * D, cache.ptr,
                            cache.size // (L * D), L * D, L, table.ptr, T, D,
                            _position_ptr(pos), x1.dtype.code))
    _wrote(x1, cache)
    return x1


def i64_add(x: DeviceTensor, delta: int):
    """x[0] += delta on the device (stream-ordered)."""
    lib_, h = _c()
    check(lib_.tl_i64_add(h, _position_ptr(x), int(delta)))
    _wrote(x)


def ids_append(ids: DeviceTensor, hist: DeviceTensor, pos: DeviceTensor, pos_base: int):
    """hist[r, *pos - pos_base] = ids[r] when that column is inside hist [rows, cols]."""
    rows, cols = hist.shape
    if ids.dtype is not int64 or hist.dtype is not int64 or ids.size != rows:
        raise ValueError("ids_append takes int64 ids [rows] and history [rows, cols]")
    lib_, h = _c()
    check(lib_.tl_ids_append(h, ids.ptr, hist.ptr, rows, hist.pitch, cols, _position_ptr(pos),
                             int(pos_base)))
    _wrote(hist)


class Graph:
    """A captured sequence of this module's calls on the context stream, replayed with one
    launch. Use as `with xp.capture() as g: <calls>`, then `g.launch()`. The calls in the
    block are recorded, not run; tensors allocated inside are written on every replay."""

    def __init__(self, handle):
        self._handle, self._ctx = handle, ctx()

    def launch(self):
        if not self._handle:
            raise TLError(TL_ERR_INVALID, "graph was destroyed")
        check(self._ctx.lib.tl_graph_launch(self._ctx.handle, self._handle))

    def destroy(self):
        if self._handle:
            h, self._handle = self._handle, None
            check(self._ctx.lib.tl_graph_destroy(self._ctx.handle, h))

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class capture:  # noqa: N801  (used as a context manager, like torch.cuda.graph)
    """with capture() as g: ... -- records the calls of the block into a Graph `g.graph`."""

    def __enter__(self):
        c = ctx()
        check(c.lib.tl_graph_begin(c.handle))
        self.graph = None
        return self

    def __exit__(self, exc_type, exc, tb):
        c = ctx()
        h = ctypes.c_void_p()
        rc = c.lib.tl_graph_end(c.handle, ctypes.byref(h))
        if exc_type is None:
            check(rc)
            self.graph = Graph(h.value)
        elif rc == TL_OK:
            c.lib.tl_graph_destroy(c.handle, h.value)
        return False

    def launch(self):
        self.graph.launch()

    def destroy(self):
        if self.graph is not None:
            self.graph.destroy()


def attention_supported(dtype, head_dim, kv_capacity) -> bool:
    """Whether tl_attention_fwd takes this configuration (bf16 with D in {32, 64, 128, 256}
    or fp32 with D in {32, 64, 128}; key capacity a multiple of 8)."""
    dt = as_dtype(dtype)
    return kv_capacity % 8 == 0 and ((dt is bfloat16 and head_dim in (32, 64, 128, 256)) or
                                     (dt is float32 and head_dim in (32, 64, 128)))


def attention_decode_dev_supported(dtype, head_dim, kv_capacity) -> bool:
    """Whether tl_attention_decode_dev takes this configuration (bf16 only)."""
    return (as_dtype(dtype) is bfloat16 and head_dim in (32, 64, 128, 256)
            and kv_capacity % 8 == 0)


def transpose2d(x: DeviceTensor, out=None, out_offset=0, ldy=None) -> DeviceTensor:
    """y[c, r] = x[r, c]. With `out`, writes into out's buffer at element `out_offset` with
    row pitch `ldy` (e.g. every other row of an interleaved pack)."""
    r, c_ = x.shape
    if out is None:
        out = DeviceTensor((c_, r), x.dtype)
        ptr, ld = out.ptr, out.pitch
    else:
        ptr, ld = out.ptr + out_offset * x.dtype.itemsize, ldy
    lib_, h = _c()
    check(lib_.tl_transpose2d(h, x.ptr, ptr, r, c_, x.pitch, ld, x.dtype.code))
    _wrote(out)
    return out


def transpose2d_gain(x: DeviceTensor, gain: DeviceTensor, gain_offset=0.0, out=None,
                     out_offset=0, ldy=None) -> DeviceTensor:
    """y[c, r] = x[r, c] * (gain_offset + gain[r]); `out`/`out_offset`/`ldy` as transpose2d."""
    r, c_ = x.shape
    if gain.size != r or gain.dtype is not x.dtype:
        raise ValueError("transpose2d_gain needs one gain of x's dtype per row of x")
    if out is None:
        out = DeviceTensor((c_, r), x.dtype)
        ptr, ld = out.ptr, out.pitch
    else:
        ptr, ld = out.ptr + out_offset * x.dtype.itemsize, ldy
    lib_, h = _c()
    check(lib_.tl_transpose2d_gain(h, x.ptr, ptr, r, c_, x.pitch, ld, gain.ptr,
                                   float(gain_offset), x.dtype.code))
    _wrote(out)
    return out


# ---- timing -------------------------------------------------------------------------------
class Event:
    def __init__(self):
        c = ctx()
        h = ctypes.c_void_p()
        check(c.lib.tl_event_create(c.handle, ctypes.byref(h)))
        self.h = h

    def record(self):
        c = ctx()
        check(c.lib.tl_event_record(c.handle, self.h))
        return self

    def elapsed_ms(self, stop: "Event") -> float:
        ms = ctypes.c_float()
        check(load_library().tl_event_elapsed_ms(self.h, stop.h, ctypes.byref(ms)))
        return ms.value

    def __del__(self):
        try:
            load_library().tl_event_destroy(self.h)
        except Exception:
            pass


def kprof_enable(families):
    mask = 0
    for f in families:
        mask |= 1 << KFAMILY[f]
    c = ctx()
    check(c.lib.tl_kprof_enable(c.handle, mask))


def kprof_reset():
    c = ctx()
    check(c.lib.tl_kprof_reset(c.handle))


def kprof_query(family):
    c = ctx()
    n, ms, fl, by = ctypes.c_int64(), ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
    check(c.lib.tl_kprof_query(c.handle, KFAMILY[family], ctypes.byref(n), ctypes.byref(ms),
                               ctypes.byref(fl), ctypes.byref(by)))
    return {"launches": n.value, "ms": ms.value, "flops": fl.value, "bytes": by.value}

