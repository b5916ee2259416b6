"""Python binding of libwgx (include/wgx.h) over ctypes.

Mirrors the reference's host API for the hot path with Python naming:
``Context`` is WgpuExecutionContext (src/context.ts:17-390), ``Tensor`` is the
non-owning view of src/tensor.ts:43-159, and the ``record_*`` methods are the
``recordIn`` bodies of the Shader objects (src/shaders/mm/index.ts:32-93,
src/shaders/bmm/index.ts:27-96, src/shaders/convolution/index.ts:58-310),
plus ``addmm`` (absent from the reference).

There is no fallback: if libwgx.so is missing or the device is absent the
calls raise.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libwgx.so")

MAX_NDIM = 8
FLOAT32, FLOAT16, INT32, INT8, UINT8, BOOL, FLOAT64, INT64, BFLOAT16 = range(9)
DTYPES = {"float32": FLOAT32, "float16": FLOAT16, "int32": INT32, "int8": INT8, "uint8": UINT8,
          "bool": BOOL, "float64": FLOAT64, "int64": INT64, "bfloat16": BFLOAT16}
DTYPE_BYTESIZE = {"float32": 4, "float16": 2, "float64": 8, "int32": 4, "int64": 8, "int8": 1,
                  "uint8": 1, "bool": 1, "bfloat16": 2}
_NP = {"float32": np.float32, "float16": np.float16, "float64": np.float64, "int32": np.int32,
       "int64": np.int64, "int8": np.int8, "uint8": np.uint8, "bool": np.uint8,
       "bfloat16": np.uint16}

USAGE_COPY_SRC, USAGE_COPY_DST, USAGE_STORAGE = 0x4, 0x8, 0x80
STORAGE_USAGE = USAGE_STORAGE | USAGE_COPY_SRC | USAGE_COPY_DST
MM_TRANS_B = 0x1
UNARY = {"sigmoid": 0, "relu": 1, "hardswish": 2, "silu": 3}

ERR_INVALID, ERR_HIP, ERR_DESTROYED, ERR_NO_DEVICE, ERR_OOM = 1, 2, 3, 4, 5


class WgxError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


class CTensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_int32), ("ndim", ctypes.c_int32),
                ("shape", ctypes.c_int64 * MAX_NDIM)]


class CConvArgs(ctypes.Structure):
    _fields_ = [("stride", ctypes.c_int32 * 2), ("padding", ctypes.c_int32 * 2),
                ("dilation", ctypes.c_int32 * 2), ("output_padding", ctypes.c_int32 * 2),
                ("transposed", ctypes.c_int32), ("groups", ctypes.c_int32),
                ("has_clamp", ctypes.c_int32), ("clamp_min", ctypes.c_float),
                ("clamp_max", ctypes.c_float), ("activation", ctypes.c_int32)]


ACT_NONE, ACT_SILU = 0, 1


_LIB = None

# every symbol include/wgx.h declares, with its ctypes signature
_P = ctypes.c_void_p
_T = ctypes.POINTER(CTensor)
_I = ctypes.c_int
_U64 = ctypes.c_uint64
SIGNATURES = {
    "wgx_ctx_create": (_I, [_I, ctypes.POINTER(_P)]),
    "wgx_ctx_create_shared": (_I, [_P, ctypes.POINTER(_P)]),
    "wgx_ctx_destroy": (None, [_P]),
    "wgx_free": (_I, [_P, _P]),
    "wgx_last_error": (ctypes.c_char_p, [_P]),
    "wgx_ctx_has_device": (_I, [_P]),
    "wgx_ctx_arch": (ctypes.c_char_p, [_P]),
    "wgx_ctx_stream": (_P, [_P]),
    "wgx_alloc": (_I, [_P, _U64, ctypes.c_uint32, ctypes.POINTER(_P)]),
    "wgx_buffer_info": (_I, [_P, _P, ctypes.POINTER(_U64), ctypes.POINTER(_U64),
                             ctypes.POINTER(ctypes.c_uint32)]),
    "wgx_write": (_I, [_P, _P, _P, _U64]),
    "wgx_read": (_I, [_P, _P, _P, _U64]),
    "wgx_record_copy": (_I, [_P, _P, _P, _U64]),
    "wgx_record_mm": (_I, [_P, _T, _T, _T, _T, ctypes.c_float, ctypes.c_float, ctypes.c_uint32]),
    "wgx_mm_noalloc": (_I, [_P, _T, _T, _T, _T, ctypes.c_float, ctypes.c_float, ctypes.c_uint32]),
    "wgx_record_bmm": (_I, [_P, _T, _T, _T, ctypes.c_uint32]),
    "wgx_record_conv2d": (_I, [_P, _T, _T, _T, ctypes.POINTER(CConvArgs), _T]),
    "wgx_record_conv2d_residual": (_I, [_P, _T, _T, _T, ctypes.POINTER(CConvArgs), _T, ctypes.c_float,
                                        ctypes.c_float, _T]),
    "wgx_record_add": (_I, [_P, _T, _T, ctypes.c_float, _I, _T]),
    "wgx_record_mul": (_I, [_P, _T, _T, _T]),
    "wgx_record_unary": (_I, [_P, _I, _T, _T]),
    "wgx_record_cat": (_I, [_P, _T, _I, _I, _T]),
    "wgx_record_split": (_I, [_P, _T, _I, _T, _I]),
    "wgx_record_upsample_nearest2d": (_I, [_P, _T, _T]),
    "wgx_record_max_pool2d": (_I, [_P, _T, ctypes.POINTER(ctypes.c_int32),
                                   ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32),
                                   ctypes.POINTER(ctypes.c_int32), _I, _T, _T]),
    "wgx_record_permute": (_I, [_P, _T, ctypes.POINTER(ctypes.c_int32), _I, _T]),
    "wgx_record_softmax": (_I, [_P, _T, _I, _T]),
    "wgx_submit": (_I, [_P]),
    "wgx_sync": (_I, [_P]),
    "wgx_fence_record": (_I, [_P, ctypes.POINTER(_P)]),
    "wgx_fence_wait": (_I, [_P]),
    "wgx_fence_error": (ctypes.c_char_p, [_P]),
    "wgx_fence_destroy": (None, [_P]),
    "wgx_reset": (_I, [_P]),
    "wgx_command_count": (_I, [_P]),
    "wgx_set_graph_mode": (_I, [_P, _I]),
    "wgx_time_submits": (_I, [_P, _I, ctypes.POINTER(ctypes.c_float)]),
    "wgx_last_kernel": (ctypes.c_char_p, [_P]),
    "wgx_paired_launches": (ctypes.c_int, [_P]),
}


def lib():
    """Load libwgx.so (built in-tree by build.py); raises if it is missing."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"libwgx.so not found at {LIB_PATH}: build it first "
                               "(python -c 'import __graft_entry__ as g; g.build()')")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


class Tensor:
    """Non-owning view: dtype + shape over a context-owned device buffer."""

    def __init__(self, ctx: "Context", dtype: str, shape: Sequence[int], ptr: int, capacity: int):
        shape = list(shape)
        if len(shape) > MAX_NDIM:
            raise ValueError(f"Tensor rank {len(shape)} exceeds maximum rank of {MAX_NDIM}")
        if any((not isinstance(d, (int, np.integer))) or d <= 0 for d in shape):
            raise ValueError("Tensor dimensions must be positive integers")
        self.ctx, self.dtype, self.shape, self.ptr = ctx, dtype, [int(d) for d in shape], int(ptr)
        self.numel = int(np.prod(self.shape)) if self.shape else 1
        self.byte_length = self.numel * DTYPE_BYTESIZE[dtype]
        if capacity < self.byte_length:
            raise ValueError(f"buffer size ({capacity}B) < required ({self.byte_length}B)")

    def c(self) -> CTensor:
        t = CTensor()
        t.data = self.ptr
        t.dtype = DTYPES[self.dtype]
        t.ndim = len(self.shape)
        for i, d in enumerate(self.shape):
            t.shape[i] = d
        return t

    def set_data(self, arr) -> "Tensor":
        """Upload host data (a prefix if smaller), like Tensor.setData."""
        a = np.ascontiguousarray(arr)
        if a.nbytes > self.byte_length:
            raise ValueError(f"setData: source {a.nbytes}B > tensor {self.byte_length}B; pass a view")
        self.ctx._check(lib().wgx_write(self.ctx.h, self.ptr, a.ctypes.data, a.nbytes))
        return self

    def get_data(self) -> np.ndarray:
        """Read back (waits for submitted work) as a numpy array of the storage type."""
        out = np.empty(self.numel, dtype=_NP[self.dtype])
        self.ctx._check(lib().wgx_read(self.ctx.h, self.ptr, out.ctypes.data, self.byte_length))
        return out.reshape(self.shape)

    def get_f32(self) -> np.ndarray:
        a = self.get_data()
        if self.dtype == "bfloat16":
            return (a.astype(np.uint32) << 16).view(np.float32)
        return a.astype(np.float32)


class Context:
    """WgpuExecutionContext over one HIP device (device=-1: host-only validation)."""

    def __init__(self, device: int = 0, _parent: Optional["Context"] = None):
        h = ctypes.c_void_p()
        if _parent is None:
            r = lib().wgx_ctx_create(device, ctypes.byref(h))
        else:
            r = lib().wgx_ctx_create_shared(_parent.h, ctypes.byref(h))
        if r != 0:
            raise WgxError(r, f"wgx_ctx_create({device}) failed with status {r}")
        self.h = h
        self.destroyed = False

    def shared(self) -> "Context":
        """A further context on this context's device: same stream and buffer
        registry, its own command list (several WgpuExecutionContexts over
        one GPUDevice)."""
        return Context(_parent=self)

    # ------------------------------------------------------------ plumbing
    def _check(self, r: int):
        if r != 0:
            raise WgxError(r, lib().wgx_last_error(self.h).decode())

    @property
    def has_device(self) -> bool:
        return bool(lib().wgx_ctx_has_device(self.h))

    @property
    def arch(self) -> str:
        return lib().wgx_ctx_arch(self.h).decode()

    @property
    def stream(self) -> int:
        return lib().wgx_ctx_stream(self.h) or 0

    @property
    def last_kernel(self) -> str:
        return lib().wgx_last_kernel(self.h).decode()

    @property
    def command_count(self) -> int:
        return lib().wgx_command_count(self.h)

    @property
    def paired_launches(self) -> int:
        """Paired convolution launches the last submit issued."""
        return lib().wgx_paired_launches(self.h)

    def destroy(self):
        if not self.destroyed:
            lib().wgx_ctx_destroy(self.h)
            self.destroyed = True

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass

    # ------------------------------------------------------------ buffers
    def storage_buffer(self, size: int, usage: int = STORAGE_USAGE) -> int:
        p = ctypes.c_void_p()
        self._check(lib().wgx_alloc(self.h, int(size), usage, ctypes.byref(p)))
        return p.value

    def free(self, ptr: int):
        """GPUBuffer.destroy(): later submits of commands that use it fail."""
        self._check(lib().wgx_free(self.h, ptr))

    def buffer_size(self, ptr: int) -> int:
        off, size = ctypes.c_uint64(), ctypes.c_uint64()
        if lib().wgx_buffer_info(self.h, ptr, ctypes.byref(off), ctypes.byref(size), None) != 0:
            raise WgxError(ERR_INVALID, "not an owned buffer")
        return size.value - off.value

    def tensor(self, dtype: str, shape: Sequence[int], buffer: Optional[int] = None) -> Tensor:
        if buffer is None:
            n = int(np.prod(shape)) if len(shape) else 1
            if len(shape) > MAX_NDIM or any(int(d) <= 0 for d in shape):
                Tensor(self, dtype, shape, 0, 0)  # raises the reference's message
            buffer = self.storage_buffer(n * DTYPE_BYTESIZE[dtype])
        return Tensor(self, dtype, shape, buffer, self.buffer_size(buffer))

    def from_numpy(self, arr: np.ndarray, dtype: Optional[str] = None) -> Tensor:
        a = np.ascontiguousarray(arr)
        if dtype is None:
            dtype = {np.float32: "float32", np.float16: "float16"}[a.dtype.type]
        if dtype == "float16":
            a = a.astype(np.float16)
        elif dtype == "float32":
            a = a.astype(np.float32)
        elif dtype == "bfloat16":
            a = f32_to_bf16_bits(a.astype(np.float32))
        t = self.tensor(dtype, a.shape if a.ndim else [1])
        return t.set_data(a)

    # ------------------------------------------------------------ records
    def copy(self, src: Tensor, dst: Tensor) -> "Context":
        if dst.byte_length < src.byte_length:
            raise ValueError(f"copy: destination ({dst.byte_length}B) < source ({src.byte_length}B)")
        self._check(lib().wgx_record_copy(self.h, dst.ptr, src.ptr, src.byte_length))
        return self

    def mm(self, a: Tensor, b: Tensor, out: Tensor, bias: Optional[Tensor] = None,
           alpha: float = 1.0, beta: float = 1.0, trans_b: bool = False) -> "Context":
        ct = [a.c(), b.c(), out.c()]
        cb = bias.c() if bias is not None else None
        self._check(lib().wgx_record_mm(self.h, ctypes.byref(ct[0]), ctypes.byref(ct[1]),
                                        ctypes.byref(cb) if cb is not None else None,
                                        ctypes.byref(ct[2]), alpha, beta,
                                        MM_TRANS_B if trans_b else 0))
        return self

    def mm_noalloc(self, a: Tensor, b: Tensor, out: Tensor, bias: Optional[Tensor] = None,
                   alpha: float = 1.0, beta: float = 1.0, trans_b: bool = False) -> "Context":
        """The mm / addmm launched now on the context's stream, its workspace in
        the library's fixed per-device scratch (no device allocation)."""
        ct = [a.c(), b.c(), out.c()]
        cb = bias.c() if bias is not None else None
        self._check(lib().wgx_mm_noalloc(self.h, ctypes.byref(ct[0]), ctypes.byref(ct[1]),
                                         ctypes.byref(cb) if cb is not None else None,
                                         ctypes.byref(ct[2]), alpha, beta,
                                         MM_TRANS_B if trans_b else 0))
        return self

    def addmm(self, bias: Tensor, x: Tensor, w: Tensor, out: Tensor, beta: float = 1.0,
              alpha: float = 1.0, trans_b: bool = False) -> "Context":
        return self.mm(x, w, out, bias=bias, alpha=alpha, beta=beta, trans_b=trans_b)

    def bmm(self, a: Tensor, b: Tensor, out: Tensor, trans_b: bool = False) -> "Context":
        ct = [a.c(), b.c(), out.c()]
        self._check(lib().wgx_record_bmm(self.h, *[ctypes.byref(t) for t in ct],
                                         MM_TRANS_B if trans_b else 0))
        return self

    def convolution(self, x: Tensor, w: Tensor, bias: Optional[Tensor], stride=(1, 1),
                    padding=(0, 0), dilation=(1, 1), transposed=False, output_padding=(0, 0),
                    groups=1, out: Optional[Tensor] = None, clamp=None, activation: int = ACT_NONE,
                    residual: Optional[Tensor] = None, conv_scale: float = 1.0,
                    residual_scale: float = 1.0) -> "Context":
        """residual: out = conv_scale * conv + residual_scale * residual (depthwise
        convolutions and the dense 3x3 ones the LDS-patch kernel takes)."""
        def hw(v):
            v = list(v) if isinstance(v, (list, tuple)) else [v]
            if len(v) == 1:
                return [v[0], v[0]]
            if len(v) == 2:
                return v
            raise ValueError("convolution: list args must be 1 or 2 elements")
        a = CConvArgs()
        a.stride[:] = hw(stride)
        a.padding[:] = hw(padding)
        a.dilation[:] = hw(dilation)
        a.output_padding[:] = hw(output_padding)
        a.transposed = int(bool(transposed))
        a.groups = int(groups)
        if clamp is not None:
            a.has_clamp = 1
            a.clamp_min = -np.inf if clamp[0] is None else float(clamp[0])
            a.clamp_max = np.inf if clamp[1] is None else float(clamp[1])
        a.activation = int(activation)
        cx, cw, co = x.c(), w.c(), out.c()
        cb = bias.c() if bias is not None else None
        if residual is not None:
            cr = residual.c()
            self._check(lib().wgx_record_conv2d_residual(self.h, ctypes.byref(cx), ctypes.byref(cw),
                                                         ctypes.byref(cb) if cb is not None else None,
                                                         ctypes.byref(a), ctypes.byref(cr), conv_scale,
                                                         residual_scale, ctypes.byref(co)))
            return self
        self._check(lib().wgx_record_conv2d(self.h, ctypes.byref(cx), ctypes.byref(cw),
                                            ctypes.byref(cb) if cb is not None else None,
                                            ctypes.byref(a), ctypes.byref(co)))
        return self

    def add(self, a: Tensor, b: Tensor, out: Tensor, alpha: float = 1.0, subtract=False):
        ca, cb, co = a.c(), b.c(), out.c()
        self._check(lib().wgx_record_add(self.h, ctypes.byref(ca), ctypes.byref(cb), alpha,
                                         int(subtract), ctypes.byref(co)))
        return self

    def mul(self, a: Tensor, b: Tensor, out: Tensor):
        ca, cb, co = a.c(), b.c(), out.c()
        self._check(lib().wgx_record_mul(self.h, ctypes.byref(ca), ctypes.byref(cb), ctypes.byref(co)))
        return self

    def unary(self, op: str, x: Tensor, out: Tensor):
        cx, co = x.c(), out.c()
        self._check(lib().wgx_record_unary(self.h, UNARY[op], ctypes.byref(cx), ctypes.byref(co)))
        return self

    def cat(self, inputs: Sequence[Tensor], dim: int, out: Tensor):
        arr = (CTensor * len(inputs))(*[t.c() for t in inputs])
        co = out.c()
        self._check(lib().wgx_record_cat(self.h, arr, len(inputs), dim, ctypes.byref(co)))
        return self

    def split(self, x: Tensor, dim: int, outputs: Sequence[Tensor]):
        arr = (CTensor * len(outputs))(*[t.c() for t in outputs])
        cx = x.c()
        self._check(lib().wgx_record_split(self.h, ctypes.byref(cx), dim, arr, len(outputs)))
        return self

    def upsample_nearest2d(self, x: Tensor, out: Tensor):
        cx, co = x.c(), out.c()
        self._check(lib().wgx_record_upsample_nearest2d(self.h, ctypes.byref(cx), ctypes.byref(co)))
        return self

    def max_pool2d(self, x: Tensor, kernel, stride, padding, dilation, out: Tensor,
                   indices: Optional[Tensor] = None, ceil_mode: bool = False):
        """max_pool2d_with_indices: values into out, int32 indices (if given)."""
        def arr(v):
            return (ctypes.c_int32 * 2)(*v)
        cx, co = x.c(), out.c()
        ci = indices.c() if indices is not None else None
        self._check(lib().wgx_record_max_pool2d(self.h, ctypes.byref(cx), arr(kernel), arr(stride),
                                                arr(padding), arr(dilation), int(bool(ceil_mode)),
                                                ctypes.byref(co),
                                                ctypes.byref(ci) if ci is not None else None))
        return self

    def permute(self, x: Tensor, dims: Sequence[int], out: Tensor):
        """permute_copy: out dim k is input dim dims[k]."""
        cx, co = x.c(), out.c()
        d = (ctypes.c_int32 * max(1, len(dims)))(*dims)
        self._check(lib().wgx_record_permute(self.h, ctypes.byref(cx), d, len(dims), ctypes.byref(co)))
        return self

    def softmax(self, x: Tensor, dim: int, out: Tensor):
        cx, co = x.c(), out.c()
        self._check(lib().wgx_record_softmax(self.h, ctypes.byref(cx), int(dim), ctypes.byref(co)))
        return self

    # ------------------------------------------------------------ execution
    def submit(self):
        self._check(lib().wgx_submit(self.h))

    def sync(self):
        self._check(lib().wgx_sync(self.h))

    def fence(self) -> int:
        """Marks the queue's current end; wait_fence(f) may run on any thread."""
        f = ctypes.c_void_p()
        self._check(lib().wgx_fence_record(self.h, ctypes.byref(f)))
        return f.value or 0

    @staticmethod
    def wait_fence(f: int, destroy: bool = True):
        try:
            r = lib().wgx_fence_wait(f)
            if r != 0:
                raise WgxError(r, lib().wgx_fence_error(f).decode())
        finally:
            if destroy:
                lib().wgx_fence_destroy(f)

    def reset(self):
        self._check(lib().wgx_reset(self.h))

    def set_graph_mode(self, enabled: bool):
        self._check(lib().wgx_set_graph_mode(self.h, int(enabled)))

    def time_submits(self, reps: int) -> float:
        ms = ctypes.c_float()
        self._check(lib().wgx_time_submits(self.h, reps, ctypes.byref(ms)))
        return ms.value


# ---------------------------------------------------------------- number formats
def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bits, round to nearest even (NaN kept quiet)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
