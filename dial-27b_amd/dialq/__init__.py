"""ctypes front end of libdialq.so (include/dialq.h) for tests and the benchmark.

The library is the product: every call below goes through the C ABI into
the HIP kernels.  There is no CPU fallback -- if the shared library is
missing, importing this module raises.

Device buffers are torch tensors on a ROCm device (torch is used only for
device memory and streams); host buffers are numpy arrays.
"""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(_HERE)
LIB_PATH = os.path.join(PKG_ROOT, "lib", "libdialq.so")
HEADER_PATH = os.path.join(PKG_ROOT, "..", "include", "dialq.h")

# enum dialq_format
W8A16, Q8_0, Q4_K, FP8_ROW, FP8_BLOCK, NVFP4, MXFP4, Q6_K = 1, 2, 3, 4, 5, 6, 7, 8
FORMAT_NAMES = {W8A16: "w8a16", Q8_0: "q8_0", Q4_K: "q4_k", FP8_ROW: "fp8_row",
                FP8_BLOCK: "fp8_block", NVFP4: "nvfp4", MXFP4: "mxfp4", Q6_K: "q6_k"}
# enum dialq_dtype
F32, F16, BF16 = 0, 1, 2
# flags
FLAG_GLOBAL_IS_DIVISOR = 0x1
FLAG_WEIGHT_ONLY_PREFILL = 0x2
# enum dialq_path
PATH_AUTO, PATH_GEMV, PATH_GEMM, PATH_GEMM_NATIVE = 0, 1, 2, 3
SELECT_FIRST_MAX, SELECT_TOTAL_LAST_MAX = 0, 1
SELECT_MAX_K = 256


class Desc(C.Structure):
    _fields_ = [("format", C.c_int32), ("scale_dtype", C.c_int32), ("out_dim", C.c_int64),
                ("in_dim", C.c_int64), ("global_scale", C.c_float), ("flags", C.c_int32)]


class DialqError(RuntimeError):
    pass


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run `python dial-27b_amd/build.py` "
                          "(or __graft_entry__.build()) first")
    # One HIP runtime per process: torch ships its own libamdhip64.so.7.  Load
    # it first so libdialq's libamdhip64.so.7 dependency resolves to the same
    # runtime (device pointers and streams are shared with the caller).  A
    # caller without torch gets /opt/rocm's runtime through the library's
    # RUNPATH.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    L = C.CDLL(LIB_PATH)
    P, I64, I32, SZ, CH = C.c_void_p, C.c_int64, C.c_int32, C.c_size_t, C.c_char_p
    sigs = {
        "dialq_abi_version": (C.c_uint32, []),
        "dialq_linear_create": (P, [C.POINTER(Desc), P, SZ, P, SZ, C.c_int, C.c_int, P, CH, SZ]),
        "dialq_linear_quantize": (P, [C.POINTER(Desc), P, I32, C.c_int, C.c_int, P, CH, SZ]),
        "dialq_linear_destroy": (None, [P]),
        "dialq_linear_resident_bytes": (C.c_uint64, [P]),
        "dialq_linear_device_bytes": (C.c_uint64, [P]),
        "dialq_linear_describe": (C.c_int, [P, C.POINTER(Desc)]),
        "dialq_linear_forward": (C.c_int, [P, P, I32, I64, P, I32, P, C.c_int, CH, SZ]),
        "dialq_linear_forward_ex": (C.c_int, [P, P, I32, I64, P, I32, I32, P, C.c_int, CH, SZ]),
        "dialq_linear_dequantize": (C.c_int, [P, P, I32, P, C.c_int, CH, SZ]),
        "dialq_linear_export": (C.c_int, [P, P, SZ, P, SZ, CH, SZ]),
        "dialq_linear_forward_swiglu": (C.c_int, [P, P, I32, I64, P, I32, I32, P, C.c_int, CH, SZ]),
        "dialq_local_q8_forward": (C.c_int, [P, P, I32, I64, P, I32, P, C.c_int, CH, SZ]),
        "dialq_logits_select_workspace_bytes": (SZ, [I64, I64]),
        "dialq_logits_select": (C.c_int, [P, I32, I64, P, I64, C.c_float, C.c_float, I32, I64, P, P, P, P, SZ,
                                          I32, P, C.c_int, CH, SZ]),
        "dialq_debug_set_wait_limit": (None, [I64]),
        "dialq_debug_grouped_launches": (I64, []),
        "dialq_linear_forward_noalloc": (C.c_int, [P, P, I32, I64, P, I32, I32, P, CH, SZ]),
        "dialq_linear_forward_group": (C.c_int, [P, I32, P, I32, I64, P, I32, I32, P, C.c_int, CH, SZ]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    return L


lib = _load()


def declared_symbols() -> list[str]:
    """Function names declared in include/dialq.h."""
    text = open(HEADER_PATH).read()
    return sorted(set(re.findall(r"\b(dialq_[a-z0-9_]+)\s*\(", text)))


def abi_version() -> int:
    return int(lib.dialq_abi_version())


def _err():
    return C.create_string_buffer(512)


def _check(rc, err):
    if rc != 0:
        raise DialqError(err.value.decode())


# ---- buffer helpers ----------------------------------------------------------
def _is_torch(a):
    return type(a).__module__.startswith("torch")


def _ptr(a):
    if a is None:
        return None
    if _is_torch(a):
        return C.c_void_p(a.data_ptr())
    a = np.ascontiguousarray(a)
    return a.ctypes.data_as(C.c_void_p)


def _nbytes(a):
    if a is None:
        return 0
    if _is_torch(a):
        return a.numel() * a.element_size()
    return np.asarray(a).nbytes


_TORCH_DT = None


def dtype_code(a) -> int:
    if _is_torch(a):
        import torch
        return {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}[a.dtype]
    a = np.asarray(a)
    if a.dtype == np.float32:
        return F32
    if a.dtype == np.float16:
        return F16
    raise ValueError(f"unsupported host dtype {a.dtype} (bf16 host arrays: pass dtype explicitly)")


def _stream_ptr(stream):
    if stream is None:
        return None
    return C.c_void_p(stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream))


class Linear:
    """Owned handle around a resident quantized weight."""

    def __init__(self, handle, desc: Desc, device: int):
        self.h = C.c_void_p(handle)
        self.desc = desc
        self.device = device

    # ---- constructors --------------------------------------------------------
    @classmethod
    def create(cls, fmt, out_dim, in_dim, weight, scales=None, *, scale_dtype=F32,
               global_scale=1.0, flags=0, device=0, stream=None):
        """Upload pre-quantized raw-format bytes (host numpy or device torch)."""
        d = Desc(fmt, scale_dtype, out_dim, in_dim, float(global_scale), flags)
        host = not _is_torch(weight)
        if host:
            weight = np.ascontiguousarray(weight)
            scales = None if scales is None else np.ascontiguousarray(scales)
        err = _err()
        h = lib.dialq_linear_create(C.byref(d), _ptr(weight), _nbytes(weight), _ptr(scales),
                                    _nbytes(scales), device, int(host), _stream_ptr(stream), err, 512)
        if not h:
            raise DialqError(err.value.decode())
        return cls(h, d, device)

    @classmethod
    def quantize(cls, fmt, dense, *, scale_dtype=F32, flags=0, device=0, stream=None,
                 dense_dtype=None):
        """Quantize a dense [N, K] weight on the GPU (host numpy or device torch)."""
        if dense_dtype is None:
            dense_dtype = dtype_code(dense)
        host = not _is_torch(dense)
        if host:
            dense = np.ascontiguousarray(dense)
        n, k = dense.shape
        d = Desc(fmt, scale_dtype, n, k, 1.0, flags)
        err = _err()
        h = lib.dialq_linear_quantize(C.byref(d), _ptr(dense), dense_dtype, device, int(host),
                                      _stream_ptr(stream), err, 512)
        if not h:
            raise DialqError(err.value.decode())
        return cls(h, d, device)

    def close(self):
        if self.h:
            lib.dialq_linear_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- properties ----------------------------------------------------------
    @property
    def out_dim(self):
        return self.desc.out_dim

    @property
    def in_dim(self):
        return self.desc.in_dim

    def resident_bytes(self) -> int:
        return int(lib.dialq_linear_resident_bytes(self.h))

    def device_bytes(self) -> int:
        return int(lib.dialq_linear_device_bytes(self.h))

    # ---- compute -------------------------------------------------------------
    def forward(self, x, y, rows=None, *, path=PATH_AUTO, stream=None, x_dtype=None, y_dtype=None):
        """y = x W^T.  torch tensors -> device pointers; numpy -> host staging."""
        dev = _is_torch(x)
        if rows is None:
            rows = (x.numel() if dev else np.asarray(x).size) // self.in_dim
        xd = dtype_code(x) if x_dtype is None else x_dtype
        yd = dtype_code(y) if y_dtype is None else y_dtype
        err = _err()
        rc = lib.dialq_linear_forward_ex(self.h, _ptr(x), xd, rows, _ptr(y), yd, path,
                                         _stream_ptr(stream), int(dev), err, 512)
        _check(rc, err)
        return y

    def forward_noalloc(self, x, y, rows=None, *, path=PATH_AUTO, stream=None, x_dtype=None, y_dtype=None):
        """dialq_linear_forward_noalloc: the same product with the library's
        static per-device scratch (device tensors only; nothing allocated)."""
        if rows is None:
            rows = x.numel() // self.in_dim
        xd = dtype_code(x) if x_dtype is None else x_dtype
        yd = dtype_code(y) if y_dtype is None else y_dtype
        err = _err()
        rc = lib.dialq_linear_forward_noalloc(self.h, _ptr(x), xd, rows, _ptr(y), yd, path, _stream_ptr(stream),
                                              err, 512)
        _check(rc, err)
        return y

    def forward_swiglu(self, x, y, rows=None, *, path=PATH_AUTO, stream=None, x_dtype=None, y_dtype=None):
        """y[:, j] = silu(x W[j]^T) * (x W[N/2 + j]^T) for a fused gate_up
        weight (gate rows first); y has out_dim / 2 columns."""
        dev = _is_torch(x)
        if rows is None:
            rows = (x.numel() if dev else np.asarray(x).size) // self.in_dim
        xd = dtype_code(x) if x_dtype is None else x_dtype
        yd = dtype_code(y) if y_dtype is None else y_dtype
        err = _err()
        rc = lib.dialq_linear_forward_swiglu(self.h, _ptr(x), xd, rows, _ptr(y), yd, path,
                                             _stream_ptr(stream), int(dev), err, 512)
        _check(rc, err)
        return y

    def local_q8(self, x, y, *, stream=None, x_dtype=None, y_dtype=None):
        dev = _is_torch(x)
        xd = dtype_code(x) if x_dtype is None else x_dtype
        yd = dtype_code(y) if y_dtype is None else y_dtype
        rows = (x.numel() if dev else np.asarray(x).size) // self.in_dim
        err = _err()
        rc = lib.dialq_local_q8_forward(self.h, _ptr(x), xd, rows, _ptr(y), yd,
                                        _stream_ptr(stream), int(dev), err, 512)
        _check(rc, err)
        return y

    def dequantize(self, out, *, stream=None, out_dtype=None):
        dev = _is_torch(out)
        od = dtype_code(out) if out_dtype is None else out_dtype
        err = _err()
        rc = lib.dialq_linear_dequantize(self.h, _ptr(out), od, _stream_ptr(stream), int(dev), err, 512)
        _check(rc, err)
        return out

    def export(self):
        """Raw-format bytes (weight, scales) as numpy arrays."""
        d = self.desc
        n, k = d.out_dim, d.in_dim
        fmt = d.format
        if fmt == W8A16:
            w = np.empty((n, k), np.int8)
            s = np.empty(n, np.uint16 if d.scale_dtype == BF16 else np.float32)
        elif fmt == Q8_0:
            w, s = np.empty((n, k // 32 * 34), np.uint8), None
        elif fmt == Q4_K:
            w, s = np.empty((n, k // 256 * 144), np.uint8), None
        elif fmt == Q6_K:
            w, s = np.empty((n, k // 256 * 210), np.uint8), None
        elif fmt == FP8_ROW:
            w, s = np.empty((n, k), np.uint8), np.empty(n, np.float32)
        elif fmt == FP8_BLOCK:
            w, s = np.empty((n, k), np.uint8), np.empty(((n + 127) // 128, (k + 127) // 128), np.float32)
        elif fmt == NVFP4:
            w, s = np.empty((n, k // 2), np.uint8), np.empty((n, k // 16), np.uint8)
        else:
            w, s = np.empty((n, k // 2), np.uint8), np.empty((n, k // 32), np.uint8)
        err = _err()
        rc = lib.dialq_linear_export(self.h, _ptr(w), w.nbytes, _ptr(s), 0 if s is None else s.nbytes,
                                     err, 512)
        _check(rc, err)
        return w, s


def forward_group(linears, x, y, rows=None, *, path=PATH_AUTO, stream=None, x_dtype=None, y_dtype=None):
    """dialq_linear_forward_group: y = cat([x W_j^T for each handle], -1),
    y of shape [rows, sum of out_dim]."""
    dev = _is_torch(x)
    k = linears[0].in_dim
    if rows is None:
        rows = (x.numel() if dev else np.asarray(x).size) // k
    xd = dtype_code(x) if x_dtype is None else x_dtype
    yd = dtype_code(y) if y_dtype is None else y_dtype
    hs = (C.c_void_p * len(linears))(*[l.h.value for l in linears])
    err = _err()
    rc = lib.dialq_linear_forward_group(hs, len(linears), _ptr(x), xd, rows, _ptr(y), yd, path,
                                        _stream_ptr(stream), int(dev), err, 512)
    _check(rc, err)
    return y


def grouped_launches():
    """Test hook (dialq_debug_grouped_launches): grouped decode and prefill launches so far."""
    return int(lib.dialq_debug_grouped_launches())


def set_wait_limit(polls):
    """Test hook (dialq_debug_set_wait_limit): polls without progress before
    the decode work queue's waits give up; negative restores the default."""
    lib.dialq_debug_set_wait_limit(int(polls))


def logits_select(logits, k=1, *, rule=SELECT_FIRST_MAX, repeat_ids=(), repeat_penalty=1.0, temperature=0.0,
                  dtype=None, workspace=None, device=0, stream=None):
    """Device token selection over one row of logits (dialq_logits_select).

    logits: a torch device tensor (asynchronous; outputs are device tensors)
    or a host numpy array (synchronous; outputs are numpy).  Returns
    (indices uint32 [k], logits f32 [k], stats f32 [2] = (max, sum) of the
    temperature-scaled softmax)."""
    dev = _is_torch(logits)
    vocab = logits.numel() if dev else np.asarray(logits).size
    ld = dtype_code(logits) if dtype is None else dtype
    ids = np.ascontiguousarray(np.asarray(list(repeat_ids), dtype=np.uint32))
    if dev:
        import torch
        out_idx = torch.empty(k, dtype=torch.int32, device=logits.device)
        out_val = torch.empty(k, dtype=torch.float32, device=logits.device)
        out_stats = torch.empty(2, dtype=torch.float32, device=logits.device)
    else:
        out_idx = np.empty(k, np.uint32)
        out_val = np.empty(k, np.float32)
        out_stats = np.empty(2, np.float32)
    err = _err()
    rc = lib.dialq_logits_select(_ptr(logits), ld, vocab, _ptr(ids) if ids.size else None, ids.size,
                                 float(repeat_penalty), float(temperature), rule, k, _ptr(out_idx), _ptr(out_val),
                                 _ptr(out_stats), _ptr(workspace), _nbytes(workspace), device,
                                 _stream_ptr(stream), int(dev), err, 512)
    _check(rc, err)
    return out_idx, out_val, out_stats


def logits_select_workspace_bytes(vocab, n_repeat=0) -> int:
    return int(lib.dialq_logits_select_workspace_bytes(vocab, n_repeat))


def raw_weight_bytes(fmt, n, k) -> int:
    """Algorithmic weight bytes of a format (packed codes + scales)."""
    if fmt == W8A16:
        return n * k + 2 * n
    if fmt == Q8_0:
        return n * (k // 32) * 34
    if fmt == Q4_K:
        return n * (k // 256) * 144
    if fmt == Q6_K:
        return n * (k // 256) * 210
    if fmt == FP8_ROW:
        return n * k + 4 * n
    if fmt == FP8_BLOCK:
        return n * k + 4 * ((n + 127) // 128) * ((k + 127) // 128)
    if fmt == NVFP4:
        return n * k // 2 + n * k // 16 + 4
    if fmt == MXFP4:
        return n * k // 2 + n * k // 32
    raise ValueError(fmt)
