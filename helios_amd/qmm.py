"""Host-side mirror of the reference's quantized-linear interface over libgemma4_qmm.

The reference calls ``mlx::core::quantized_matmul(x, w, scales, biases,
transpose=true, group_size, bits, "affine")`` for every projection
(``native/gemma4_mlx/src/native_model.cc:349-362``, lm_head ``:1782-1795``) and
``mlx::core::dequantize`` for the embedding (``:364-376``).  This module offers
the same operations with the same argument meaning on device tensors:

* :func:`quantized_matmul` / :func:`dequantize` — one-shot, MLX-style signatures;
* :class:`QuantizedLinear` — the resident-weight form the call sites actually
  need (weights loaded once, ``forward`` per step), one C-ABI handle each;
* :class:`QuantizedGeGLU` — gate and up as one resident pair whose ``forward``
  returns ``geglu(x . Wg^T, x . Wu^T)``, the MLP front half of
  ``native_model.cc:934-949`` with ``geglu`` (``:378-386``) fused in.

Errors surface as :class:`Gemma4Error` carrying the C status and the native
last-error text, as the reference's Rust wrapper does with ``check()``
(``crates/gemma4d-ffi/src/lib.rs:1409-1433``).  Torch supplies device memory and
the current stream only; all arithmetic runs in the HIP kernels.  There is no
fallback: without the built library every call raises.
"""

from __future__ import annotations

import contextlib
import ctypes
import enum
import os

import numpy as np

from . import build as _build

LIB_PATH = _build.LIB_PATH


class Status(enum.IntEnum):
    """Gemma4Status (native/gemma4_mlx/include/gemma4_mlx.h:12-21)."""

    OK = 0
    INVALID_ARGUMENT = 1
    UNSUPPORTED_CONFIG = 2
    MODEL_LOAD = 3
    RUNTIME = 4
    MEMORY_GUARD = 5
    CACHE = 6
    ADAPTER = 7


class Gemma4Error(RuntimeError):
    def __init__(self, status: int, message: str):
        self.status = Status(status)
        self.message = message
        super().__init__(f"{self.status.name}: {message}")


class _Desc(ctypes.Structure):
    _fields_ = [("out_features", ctypes.c_uint32), ("in_features", ctypes.c_uint32),
                ("bits", ctypes.c_uint32), ("group_size", ctypes.c_uint32)]


class _Info(ctypes.Structure):
    _fields_ = [("out_features", ctypes.c_uint32), ("in_features", ctypes.c_uint32),
                ("bits", ctypes.c_uint32), ("group_size", ctypes.c_uint32),
                ("device_bytes", ctypes.c_uint64), ("device", ctypes.c_int32),
                ("flags", ctypes.c_uint32)]


class _Version(ctypes.Structure):
    _fields_ = [("abi_version", ctypes.c_uint32), ("backend_name", ctypes.c_char_p),
                ("backend_version", ctypes.c_char_p)]


DTYPE_BF16 = 0
DTYPE_F32 = 1
GEGLU_PAIR = 1  # Gemma4QLinearInfo.flags

_lib = None


def load_library(path: str | None = None):
    """Loads libgemma4_qmm.so (built by ``python -m helios_amd.build``), or the build
    at `path`, and makes it the library the classes and functions here call."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    try:
        # PyTorch-ROCm wheels carry their own libamdhip64 (same soname as the system
        # one this library links).  Loaded first, torch's copy also serves this library;
        # loaded after it, torch would map a second HIP runtime into the process, and
        # the runtime that initialises second finds no device.
        import torch  # noqa: F401
    except ImportError:
        pass
    path = path or LIB_PATH
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it with `python -m helios_amd.build`")
    lib = ctypes.CDLL(path)
    vp = ctypes.c_void_p
    st = ctypes.c_int
    sig = {
        "gemma4_qmm_runtime_version": [ctypes.POINTER(_Version)],
        "gemma4_qmm_get_last_error": [ctypes.c_char_p, ctypes.c_size_t],
        "gemma4_qmm_set_gemm_min_rows": [ctypes.c_uint32],
        "gemma4_qmm_set_decode_kernel": [ctypes.c_uint32],
        "gemma4_qmm_set_gemm_form": [ctypes.c_uint32],
        "gemma4_qmm_release_scratch": [vp],
        "gemma4_qlinear_scratch_bytes": [vp, ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint64)],
        "gemma4_qmlp_forward": [vp, vp, vp, vp, ctypes.c_uint32, vp, vp, ctypes.c_uint32],
        "gemma4_qlinear_create": [ctypes.POINTER(_Desc), vp, vp, vp, ctypes.POINTER(vp)],
        "gemma4_qlinear_create_device": [ctypes.POINTER(_Desc), vp, vp, vp, vp, ctypes.POINTER(vp)],
        "gemma4_qlinear_free": [vp],
        "gemma4_qlinear_info": [vp, ctypes.POINTER(_Info)],
        "gemma4_qlinear_forward": [vp, vp, vp, ctypes.c_uint32, vp, ctypes.c_int],
        "gemma4_qlinear_forward_noalloc": [vp, vp, vp, ctypes.c_uint32, vp, ctypes.c_int],
        "gemma4_qlinear_dequantize": [vp, vp, vp],
        "gemma4_qgeglu_create": [ctypes.POINTER(_Desc), vp, vp, vp, vp, vp, vp, ctypes.POINTER(vp)],
        "gemma4_qgeglu_create_device": [ctypes.POINTER(_Desc), vp, vp, vp, vp, vp, vp, vp, ctypes.POINTER(vp)],
        "gemma4_qgeglu_forward": [vp, vp, vp, ctypes.c_uint32, vp, ctypes.c_int],
        "gemma4_qlinear_forward_greedy": [vp, vp, vp, ctypes.c_uint32, ctypes.c_float, vp, ctypes.c_int, vp, vp],
        "gemma4_qlinear_embed": [vp, vp, vp, ctypes.c_uint32, vp, ctypes.c_int],
        "gemma4_qlora_create": [vp, vp, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_float,
                                ctypes.POINTER(vp)],
        "gemma4_qlora_free": [vp],
        "gemma4_qlinear_forward_lora": [vp, vp, vp, vp, ctypes.c_uint32, vp, ctypes.c_int],
    }
    for name, args in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = ctypes.c_uint32 if name.startswith("gemma4_qmm_set_") else st
    _lib = lib
    return lib


def last_error(lib=None) -> str:
    lib = lib or load_library()
    buf = ctypes.create_string_buffer(512)
    if lib.gemma4_qmm_get_last_error(buf, len(buf)) != 0:
        return "native error unavailable"
    return buf.value.decode("utf-8", "replace")


def check(status: int, lib=None) -> None:
    if status != Status.OK:
        raise Gemma4Error(status, last_error(lib))


def runtime_version() -> dict:
    lib = load_library()
    v = _Version()
    check(lib.gemma4_qmm_runtime_version(ctypes.byref(v)), lib)
    return {"abi_version": v.abi_version, "backend_name": v.backend_name.decode(),
            "backend_version": v.backend_version.decode()}


def set_gemm_min_rows(rows: int) -> int:
    """Pins the forward path for this process: 0 (the default) chooses by shape; r > 0
    runs the GEMM from r rows on and the decode kernels below.  Returns the previous
    setting."""
    if not 0 <= int(rows) < 2 ** 32:
        raise ValueError(f"rows must be in [0, 2**32), got {rows}")
    return int(load_library().gemma4_qmm_set_gemm_min_rows(int(rows)))


def release_scratch(stream=None) -> None:
    """Frees the device memory the library keeps for the scratch of calls on `stream`
    (default: torch's current stream) on the current device, after waiting for the
    stream.  Graphs captured on it that used that memory must not be replayed after."""
    lib = load_library()
    check(lib.gemma4_qmm_release_scratch(_stream_ptr(stream)), lib)


def set_decode_kernel(variant: int) -> int:
    """Pins the decode kernel family for this process: 0 (the default) chooses by
    shape, 1 the int8 matrix-core kernels for every call of 1-8 rows they can run, 2
    the bf16 kernels only.  Returns the previous setting."""
    if int(variant) not in (0, 1, 2):
        raise ValueError(f"variant must be 0, 1 or 2, got {variant}")
    return int(load_library().gemma4_qmm_set_decode_kernel(int(variant)))


def set_gemm_form(form: int) -> int:
    """Pins the GEMM form for this process: 0 (the default) the fp16 form wherever a
    handle's scales allow it, 1 the bf16 form only.  Returns the previous setting."""
    if int(form) not in (0, 1):
        raise ValueError(f"form must be 0 or 1, got {form}")
    return int(load_library().gemma4_qmm_set_gemm_form(int(form)))


@contextlib.contextmanager
def gemm_form(form: int):
    """set_gemm_form for the duration of a with-block."""
    prev = set_gemm_form(form)
    try:
        yield
    finally:
        set_gemm_form(prev)


@contextlib.contextmanager
def decode_kernel(variant: int):
    """set_decode_kernel for the duration of a with-block."""
    prev = set_decode_kernel(variant)
    try:
        yield
    finally:
        set_decode_kernel(prev)


@contextlib.contextmanager
def gemm_min_rows(rows: int):
    """set_gemm_min_rows for the duration of a with-block."""
    prev = set_gemm_min_rows(rows)
    try:
        yield
    finally:
        set_gemm_min_rows(prev)


def _stream_ptr(stream):
    import torch

    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _dev_ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def _check_spec(group_size: int, bits: int, mode: str, transpose: bool = True) -> None:
    if mode != "affine":
        raise Gemma4Error(Status.UNSUPPORTED_CONFIG, f"mode {mode!r} is not supported (affine only)")
    if not transpose:
        raise Gemma4Error(Status.UNSUPPORTED_CONFIG, "transpose=False is not supported (the call sites use y = x . W^T)")
    if bits not in (4, 8) or group_size != 64:
        raise Gemma4Error(Status.UNSUPPORTED_CONFIG,
                          f"only bits=4 or 8 with group_size=64 is supported (got bits={bits} group_size={group_size})")


def _host_triple(weight, scales, biases, n: int, k: int, group_size: int, bits: int):
    w = np.ascontiguousarray(weight, dtype=np.uint32)
    s = np.ascontiguousarray(scales, dtype=np.uint16)
    b = np.ascontiguousarray(biases, dtype=np.uint16)
    wc = k * bits // 32
    if w.shape != (n, wc) or s.shape != (n, k // group_size) or b.shape != s.shape:
        raise Gemma4Error(Status.INVALID_ARGUMENT, f"weight must be [{n}, {wc}] and scales/biases [{n}, {k // group_size}]")
    return w, s, b


def _device_triple(weight, scales, biases, n: int, k: int, group_size: int, bits: int):
    import torch

    w = weight.contiguous()
    s = scales.contiguous()
    b = biases.contiguous()
    if w.dtype not in (torch.int32, torch.uint32) or s.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
        raise Gemma4Error(Status.INVALID_ARGUMENT, "weight must be int32/uint32 and scales/biases bfloat16")
    wc = k * bits // 32
    if tuple(w.shape) != (n, wc) or tuple(s.shape) != (n, k // group_size) or tuple(b.shape) != tuple(s.shape):
        raise Gemma4Error(Status.INVALID_ARGUMENT, f"weight must be [{n}, {wc}] and scales/biases [{n}, {k // group_size}]")
    if not (w.is_cuda and s.is_cuda and b.is_cuda):
        raise Gemma4Error(Status.INVALID_ARGUMENT, "device tensors must be on a CUDA (HIP) device")
    return w, s, b


def _host_ptrs(t):
    return [a.ctypes.data_as(ctypes.c_void_p) for a in t]


def _run_forward(fn, handle, lib, x, in_features: int, out_features: int, out=None, out_dtype=None, stream=None):
    import torch

    if out_dtype is None:
        out_dtype = out.dtype if out is not None else torch.bfloat16
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise Gemma4Error(Status.INVALID_ARGUMENT, "out_dtype must be bfloat16 or float32")
    if x.dtype != torch.bfloat16:
        raise Gemma4Error(Status.INVALID_ARGUMENT, "x must be bfloat16")
    if x.shape[-1] != in_features:
        raise Gemma4Error(Status.INVALID_ARGUMENT, f"x last dim {x.shape[-1]} != in_features {in_features}")
    lead = tuple(x.shape[:-1])
    x2 = x.reshape(-1, in_features).contiguous()
    rows = x2.shape[0]
    if out is None:
        out = torch.empty(lead + (out_features,), dtype=out_dtype, device=x.device)
    elif out.dtype != out_dtype or tuple(out.shape) != lead + (out_features,) or not out.is_contiguous():
        raise Gemma4Error(Status.INVALID_ARGUMENT, "out has the wrong dtype, shape or layout")
    code = DTYPE_F32 if out_dtype == torch.float32 else DTYPE_BF16
    check(fn(handle, _stream_ptr(stream), _dev_ptr(x2), rows, _dev_ptr(out), code), lib)
    return out


class _Handle:
    """Owner of one ``Gemma4QLinear`` handle (freed by ``close`` or on collection)."""

    _handle = None

    def info(self) -> dict:
        info = _Info()
        check(self._lib.gemma4_qlinear_info(self._handle, ctypes.byref(info)), self._lib)
        return {f: getattr(info, f) for f, _ in _Info._fields_}

    def scratch_bytes(self, rows: int) -> int:
        """Scratch bytes a forward of `rows` rows takes (0 on the decode path); at most
        64 MiB means forward_noalloc runs the same plan (identical bits)."""
        out = ctypes.c_uint64(0)
        check(self._lib.gemma4_qlinear_scratch_bytes(self._handle, int(rows), ctypes.byref(out)), self._lib)
        return int(out.value)

    @property
    def device(self):
        """The torch device that holds the handle's weights (outputs allocated by
        this object go there, whatever the current device is)."""
        import torch

        return torch.device("cuda", self.info()["device"])

    def close(self) -> None:
        if getattr(self, "_handle", None) is not None and self._handle.value:
            check(self._lib.gemma4_qlinear_free(self._handle), self._lib)
            self._handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class QuantizedLinear(_Handle):
    """One projection's weight triple resident on the GPU (a ``Gemma4QLinear`` handle).

    ``weight`` uint32/int32 [N, K*bits/32], ``scales``/``biases`` bf16 [N, K/64] in
    MLX layout — torch tensors on the current CUDA device, or numpy arrays on the
    host (``uint32`` and ``uint16`` bit patterns).  bits is 4 or 8 (group 64)."""

    def __init__(self, weight, scales, biases, group_size: int = 64, bits: int = 4, stream=None):
        _check_spec(group_size, bits, "affine")
        self._lib = load_library()
        self._handle = ctypes.c_void_p()
        n = int(weight.shape[0])
        k = int(weight.shape[1]) * 32 // bits
        desc = _Desc(n, k, bits, group_size)
        if isinstance(weight, np.ndarray):
            t = _host_triple(weight, scales, biases, n, k, group_size, bits)
            status = self._lib.gemma4_qlinear_create(ctypes.byref(desc), *_host_ptrs(t), ctypes.byref(self._handle))
        else:
            import torch

            t = _device_triple(weight, scales, biases, n, k, group_size, bits)
            with torch.cuda.device(t[0].device):
                status = self._lib.gemma4_qlinear_create_device(ctypes.byref(desc), *map(_dev_ptr, t),
                                                                _stream_ptr(stream), ctypes.byref(self._handle))
        check(status, self._lib)
        self.out_features = n
        self.in_features = k
        self.group_size = group_size
        self.bits = bits

    def forward(self, x, out=None, out_dtype=None, stream=None):
        """y = x . W^T for x bf16 [..., K] on the device; returns [..., N]."""
        return _run_forward(self._lib.gemma4_qlinear_forward, self._handle, self._lib, x, self.in_features,
                            self.out_features, out, out_dtype, stream)

    __call__ = forward

    def forward_noalloc(self, x, out, stream=None):
        """forward into a caller-owned `out` through gemma4_qlinear_forward_noalloc: no
        device allocation by the library (its scratch is a static per-GPU array, so
        overlapping calls on one GPU race; see include/gemma4_qmm.h)."""
        return _run_forward(self._lib.gemma4_qlinear_forward_noalloc, self._handle, self._lib, x, self.in_features,
                            self.out_features, out, out.dtype, stream)

    def forward_raw(self, x_ptr: int, rows: int, y_ptr: int, f32: bool = False, stream_ptr: int = 0) -> None:
        """Direct C-ABI call on raw device pointers (benchmark loops)."""
        check(self._lib.gemma4_qlinear_forward(self._handle, ctypes.c_void_p(stream_ptr), ctypes.c_void_p(x_ptr),
                                               rows, ctypes.c_void_p(y_ptr), DTYPE_F32 if f32 else DTYPE_BF16),
              self._lib)

    def forward_greedy(self, x, softcap: float = 30.0, out_dtype=None, return_logits: bool = False, stream=None):
        """The greedy lm_head: softcapped logits of x . W^T and their argmax per row.

        Returns (token int32 [rows], value float32 [rows], logits [rows, N] or None):
        the first maximum of each row's tanh(logits / softcap) * softcap and that
        maximum (native_model.cc:1782-1795 and the argmax at :3734).  x is bf16
        [rows, K] with rows <= 16; softcap 0 skips the softcap."""
        import torch

        out_dtype = out_dtype or torch.bfloat16
        if out_dtype not in (torch.bfloat16, torch.float32):
            raise Gemma4Error(Status.INVALID_ARGUMENT, "out_dtype must be bfloat16 or float32")
        if x.dtype != torch.bfloat16 or x.shape[-1] != self.in_features:
            raise Gemma4Error(Status.INVALID_ARGUMENT, f"x must be bfloat16 [..., {self.in_features}]")
        x2 = x.reshape(-1, self.in_features).contiguous()
        rows = x2.shape[0]
        token = torch.empty((rows,), dtype=torch.int32, device=x.device)
        value = torch.empty((rows,), dtype=torch.float32, device=x.device)
        logits = torch.empty((rows, self.out_features), dtype=out_dtype, device=x.device) if return_logits else None
        code = DTYPE_F32 if out_dtype == torch.float32 else DTYPE_BF16
        check(self._lib.gemma4_qlinear_forward_greedy(
            self._handle, _stream_ptr(stream), _dev_ptr(x2), rows, float(softcap),
            _dev_ptr(logits) if logits is not None else None, code, _dev_ptr(token), _dev_ptr(value)), self._lib)
        return token, value, logits

    def forward_lora(self, x, lora, out=None, out_dtype=None, stream=None):
        """forward plus a LoRA adapter's delta (native_model.cc:316-328); lora None is
        the plain forward."""
        handle = lora._handle if lora is not None else None
        fn = lambda h, st, xp, rows, yp, code: self._lib.gemma4_qlinear_forward_lora(  # noqa: E731
            h, handle, st, xp, rows, yp, code)
        return _run_forward(fn, self._handle, self._lib, x, self.in_features, self.out_features, out, out_dtype, stream)

    def embed(self, ids, out_dtype=None, stream=None):
        """Rows ids of the dequantized weight, [len(ids), K] (the quantized embedding
        gather, native_model.cc:364-376).  ids: int32 device tensor; rows outside
        [0, N) come back as zeros.  fp32 is bit-exact; bf16 is it rounded once."""
        import torch

        out_dtype = out_dtype or torch.bfloat16
        if out_dtype not in (torch.bfloat16, torch.float32):
            raise Gemma4Error(Status.INVALID_ARGUMENT, "out_dtype must be bfloat16 or float32")
        ids = ids.to(torch.int32).contiguous()
        out = torch.empty((ids.numel(), self.in_features), dtype=out_dtype, device=ids.device)
        check(self._lib.gemma4_qlinear_embed(self._handle, _stream_ptr(stream), _dev_ptr(ids), ids.numel(),
                                             _dev_ptr(out), DTYPE_F32 if out_dtype == torch.float32 else DTYPE_BF16),
              self._lib)
        return out.reshape(tuple(ids.shape) + (self.in_features,))

    def dequantize(self, stream=None):
        import torch

        out = torch.empty((self.out_features, self.in_features), dtype=torch.float32, device=self.device)
        check(self._lib.gemma4_qlinear_dequantize(self._handle, _stream_ptr(stream), _dev_ptr(out)), self._lib)
        return out


class QuantizedGeGLU(_Handle):
    """Gate and up projections resident as one pair: ``forward(x)`` returns
    ``h = geglu(x . Wg^T, x . Wu^T)`` [..., F], the reference's two quantized_linear
    calls and ``geglu`` (``native_model.cc:934-949``, ``:378-386``) in one kernel.
    In bf16 the qmm outputs and each GeGLU op round to bf16 as the reference's bf16
    array ops do; in fp32 (the float32 override) everything stays fp32.  Triples as
    for :class:`QuantizedLinear`; both must have the same shape."""

    def __init__(self, gate, up, group_size: int = 64, bits: int = 4, stream=None):
        _check_spec(group_size, bits, "affine")
        self._lib = load_library()
        self._handle = ctypes.c_void_p()
        n = int(gate[0].shape[0])
        k = int(gate[0].shape[1]) * 32 // bits
        desc = _Desc(n, k, bits, group_size)
        if isinstance(gate[0], np.ndarray):
            tg = _host_triple(*gate, n, k, group_size, bits)
            tu = _host_triple(*up, n, k, group_size, bits)
            status = self._lib.gemma4_qgeglu_create(ctypes.byref(desc), *_host_ptrs(tg), *_host_ptrs(tu),
                                                    ctypes.byref(self._handle))
        else:
            import torch

            tg = _device_triple(*gate, n, k, group_size, bits)
            tu = _device_triple(*up, n, k, group_size, bits)
            with torch.cuda.device(tg[0].device):
                status = self._lib.gemma4_qgeglu_create_device(ctypes.byref(desc), *map(_dev_ptr, tg),
                                                               *map(_dev_ptr, tu), _stream_ptr(stream),
                                                               ctypes.byref(self._handle))
        check(status, self._lib)
        self.out_features = n
        self.in_features = k
        self.group_size = group_size
        self.bits = bits

    def forward(self, x, out=None, out_dtype=None, stream=None):
        """h = geglu(x . Wg^T, x . Wu^T) for x bf16 [..., K] on the device; returns [..., F]."""
        return _run_forward(self._lib.gemma4_qgeglu_forward, self._handle, self._lib, x, self.in_features,
                            self.out_features, out, out_dtype, stream)

    __call__ = forward

    def forward_mlp(self, down, x, out=None, h=None, stream=None):
        """The MLP block through gemma4_qmlp_forward: h = geglu(x . Wg^T, x . Wu^T) and
        y = h . Wd^T on the projection `down` (in_features = F), bf16 throughout (the
        reference's decode MLP, ``native_model.cc:1318-1321``).  One launch at one
        row.  Returns (y [..., N_down], h [..., F]); `out` and `h` may be given."""
        import torch

        if x.dtype != torch.bfloat16 or x.shape[-1] != self.in_features:
            raise Gemma4Error(Status.INVALID_ARGUMENT, f"x must be bfloat16 [..., {self.in_features}]")
        lead = tuple(x.shape[:-1])
        x2 = x.reshape(-1, self.in_features).contiguous()
        rows = x2.shape[0]
        if h is None:
            h = torch.empty(lead + (self.out_features,), dtype=torch.bfloat16, device=x.device)
        if out is None:
            out = torch.empty(lead + (down.out_features,), dtype=torch.bfloat16, device=x.device)
        for t, n, what in ((h, self.out_features, "h"), (out, down.out_features, "out")):
            if t.dtype != torch.bfloat16 or tuple(t.shape) != lead + (n,) or not t.is_contiguous():
                raise Gemma4Error(Status.INVALID_ARGUMENT, f"{what} has the wrong dtype, shape or layout")
        check(self._lib.gemma4_qmlp_forward(self._handle, down._handle, _stream_ptr(stream), _dev_ptr(x2), rows,
                                            _dev_ptr(h), _dev_ptr(out), DTYPE_BF16), self._lib)
        return out, h

    def forward_raw(self, x_ptr: int, rows: int, h_ptr: int, f32: bool = False, stream_ptr: int = 0) -> None:
        """Direct C-ABI call on raw device pointers (benchmark loops)."""
        check(self._lib.gemma4_qgeglu_forward(self._handle, ctypes.c_void_p(stream_ptr), ctypes.c_void_p(x_ptr),
                                              rows, ctypes.c_void_p(h_ptr), DTYPE_F32 if f32 else DTYPE_BF16),
              self._lib)

    def dequantize(self, stream=None):
        """fp32 [2, F, K]: the gate rows, then the up rows (bit-exact)."""
        import torch

        out = torch.empty((2, self.out_features, self.in_features), dtype=torch.float32, device=self.device)
        check(self._lib.gemma4_qlinear_dequantize(self._handle, _stream_ptr(stream), _dev_ptr(out)), self._lib)
        return out


class LoraAdapter:
    """One LoRA module on the current device: A [rank, K] and B [N, rank] (float32, as
    the reference casts lora_A / lora_B, native_model.cc:3420-3426) and scale =
    alpha / rank.  Used with QuantizedLinear.forward_lora."""

    def __init__(self, a, b, scale: float):
        self._lib = load_library()
        self._handle = ctypes.c_void_p()
        a = np.ascontiguousarray(a, dtype=np.float32)
        b = np.ascontiguousarray(b, dtype=np.float32)
        if a.ndim != 2 or b.ndim != 2 or b.shape[1] != a.shape[0]:
            raise Gemma4Error(Status.ADAPTER, f"LoRA shapes do not chain: A {a.shape}, B {b.shape}")
        self.rank, self.in_features = a.shape
        self.out_features = b.shape[0]
        self.scale = float(scale)
        check(self._lib.gemma4_qlora_create(a.ctypes.data_as(ctypes.c_void_p), b.ctypes.data_as(ctypes.c_void_p),
                                            self.rank, self.in_features, self.out_features, self.scale,
                                            ctypes.byref(self._handle)), self._lib)

    def close(self) -> None:
        if getattr(self, "_handle", None) is not None and self._handle.value:
            check(self._lib.gemma4_qlora_free(self._handle), self._lib)
            self._handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def quantized_matmul(x, w, scales, biases, transpose: bool = True, group_size: int = 64, bits: int = 4,
                     mode: str = "affine", out_dtype=None):
    """MLX ``quantized_matmul`` with MLX's argument meaning; returns x's dtype by default."""
    _check_spec(group_size, bits, mode, transpose)
    lin = QuantizedLinear(w, scales, biases, group_size, bits)
    try:
        return lin.forward(x, out_dtype=out_dtype)
    finally:
        lin.close()


def dequantize(w, scales, biases, group_size: int = 64, bits: int = 4, mode: str = "affine"):
    """MLX ``dequantize(..., dtype=float32)``: fp32 [N, K] with w = s*q + b."""
    _check_spec(group_size, bits, mode)
    lin = QuantizedLinear(w, scales, biases, group_size, bits)
    try:
        return lin.dequantize()
    finally:
        lin.close()
