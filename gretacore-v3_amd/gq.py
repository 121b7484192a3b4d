"""Python binding of libgq.so (the C ABI declared in include/gq.h).

Thin ctypes layer: device buffers are torch tensors on a ROCm device (torch is
only the allocator / stream provider here); every compute call goes through the
HIP kernels in libgq.so.  There is no CPU fallback: if the library is missing
or a call fails, an exception is raised.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libgq.so")

FMT_Q4_0 = 2
FMT_Q8_0 = 8
FMT_Q4_K = 12
FMT_Q4_K_GGML = 112
FORMATS = {"q4_0": FMT_Q4_0, "q8_0": FMT_Q8_0, "q4_k": FMT_Q4_K, "q4_k_ggml": FMT_Q4_K_GGML}

DT_F32, DT_F16, DT_BF16 = 0, 1, 2
MAX_BATCH = 16

_c_size = ctypes.c_size_t
_vp = ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/gq.h
_SIGS = {
    "gq_abi_version": (ctypes.c_int, []),
    "gq_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "gq_last_error": (ctypes.c_char_p, []),
    "gq_gguf_bytes": (_c_size, [ctypes.c_int, _c_size, _c_size]),
    "gq_packed_size": (ctypes.c_int, [ctypes.c_int, _c_size, _c_size, ctypes.POINTER(_c_size)]),
    "gq_repack_host": (ctypes.c_int, [ctypes.c_int, _vp, _c_size, _c_size, _vp]),
    "gq_unpack_host": (ctypes.c_int, [ctypes.c_int, _vp, _c_size, _c_size, _vp]),
    "gq_repack": (ctypes.c_int, [ctypes.c_int, _vp, _c_size, _c_size, _vp, _vp]),
    "gq_dequant_gguf": (ctypes.c_int, [ctypes.c_int, _vp, _c_size, _vp, _vp]),
    "gq_dequant_packed": (ctypes.c_int, [ctypes.c_int, _vp, _c_size, _c_size, _vp, _vp]),
    "gq_gemv_workspace_bytes": (_c_size, [ctypes.c_int, _c_size, ctypes.c_int]),
    "gq_gemv": (ctypes.c_int, [ctypes.c_int, _vp, _vp, _vp, _c_size, _c_size, ctypes.c_int, _vp, _c_size, _vp]),
    "gq_gemv_plan": (ctypes.c_int, [ctypes.c_int, _c_size, _c_size, ctypes.c_int, ctypes.POINTER(ctypes.c_int),
                                     ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]),
    "gq_gemv_prep": (ctypes.c_int, [ctypes.c_int, _vp, _c_size, ctypes.c_int, _vp, _c_size, _vp]),
    "gq_gemv_prepped": (ctypes.c_int, [ctypes.c_int, _vp, _vp, _vp, _c_size, _c_size, ctypes.c_int, _vp]),
    "gq_gemm_workspace_bytes": (_c_size, [ctypes.c_int, _c_size, _c_size]),
    "gq_gemm": (ctypes.c_int, [ctypes.c_int, _vp, _vp, ctypes.c_int, _vp, ctypes.c_int, _c_size, _c_size,
                               _c_size, _vp, _c_size, _vp]),
    "gq_quantize_act_q8": (ctypes.c_int, [_vp, ctypes.c_int, _c_size, _c_size, _vp, _vp, _vp]),
    "gq_gemm_q8_i8": (ctypes.c_int, [_vp, _vp, _vp, _vp, _c_size, _c_size, _c_size, _vp]),
    "gq_matmul": (ctypes.c_int, [ctypes.c_int, _vp, _vp, _vp, _c_size, _c_size, _c_size, _vp]),
    "gq_launch_gemm_mfma_int8_wt_fp32_acc32": (
        ctypes.c_int, [_vp, _vp, _vp, _vp, _vp] + [ctypes.c_uint32] * 7),
    "gq_launch_gemm_mfma_int4_wt_fp32_acc32": (
        ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp] + [ctypes.c_uint32] * 8 + [ctypes.c_int, ctypes.c_int]),
}

_lib = None


class GQError(RuntimeError):
    pass


def load(path: str | None = None):
    """Load libgq.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise GQError(f"libgq.so not built: {p} missing (run __graft_entry__.build())")
    lib = ctypes.CDLL(p)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def exported_symbols():
    return list(_SIGS)


def check(status: int, what: str = "gq call"):
    if status != 0:
        lib = load()
        msg = lib.gq_status_string(status).decode()
        err = lib.gq_last_error().decode()
        raise GQError(f"{what} failed: {msg} ({status}){': ' + err if err else ''}")


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _require_device(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise GQError("device tensor expected (libgq has no CPU path)")


# ---- sizes / host repack (no GPU needed) ----------------------------------
def gguf_bytes(fmt: int, n: int, k: int) -> int:
    return load().gq_gguf_bytes(fmt, n, k)


def packed_size(fmt: int, n: int, k: int) -> int:
    out = _c_size(0)
    check(load().gq_packed_size(fmt, n, k, ctypes.byref(out)), "gq_packed_size")
    return out.value


def repack_host(fmt: int, gguf, n: int, k: int):
    """numpy uint8 GGUF rows -> numpy uint8 T16 tensor."""
    import numpy as np
    src = np.ascontiguousarray(gguf, dtype=np.uint8)
    out = np.empty(packed_size(fmt, n, k), dtype=np.uint8)
    check(load().gq_repack_host(fmt, src.ctypes.data, n, k, out.ctypes.data), "gq_repack_host")
    return out


def unpack_host(fmt: int, packed, n: int, k: int):
    import numpy as np
    src = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.empty(gguf_bytes(fmt, n, k), dtype=np.uint8)
    check(load().gq_unpack_host(fmt, src.ctypes.data, n, k, out.ctypes.data), "gq_unpack_host")
    return out


# ---- device entry points ----------------------------------------------------
def repack(fmt: int, d_gguf, n: int, k: int, stream=None):
    import torch
    _require_device(d_gguf)
    out = torch.empty(packed_size(fmt, n, k), dtype=torch.uint8, device=d_gguf.device)
    check(load().gq_repack(fmt, _ptr(d_gguf), n, k, _ptr(out), _stream(stream)), "gq_repack")
    return out


def dequant_gguf(fmt: int, d_blocks, n_blocks: int, stream=None):
    import torch
    _require_device(d_blocks)
    per = 256 if fmt in (FMT_Q4_K, FMT_Q4_K_GGML) else 32
    out = torch.empty(n_blocks * per, dtype=torch.float32, device=d_blocks.device)
    check(load().gq_dequant_gguf(fmt, _ptr(d_blocks), n_blocks, _ptr(out), _stream(stream)), "gq_dequant_gguf")
    return out


def dequant_packed(fmt: int, d_packed, n: int, k: int, stream=None):
    import torch
    _require_device(d_packed)
    out = torch.empty((n, k), dtype=torch.float32, device=d_packed.device)
    check(load().gq_dequant_packed(fmt, _ptr(d_packed), n, k, _ptr(out), _stream(stream)), "gq_dequant_packed")
    return out


class Workspace:
    """Caller-owned device workspace reused across calls."""

    def __init__(self, device, nbytes: int = 0):
        self.device = device
        self.buf = None
        self.ensure(nbytes)

    def ensure(self, nbytes: int):
        import torch
        if self.buf is None or self.buf.numel() < nbytes:
            self.buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=self.device)
        return self.buf


def gemv_plan(fmt: int, n: int, k: int, batch: int):
    """(row tiles per workgroup, waves per workgroup, max chunks per wave)."""
    r, ks, cpw = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    check(load().gq_gemv_plan(fmt, n, k, batch, ctypes.byref(r), ctypes.byref(ks), ctypes.byref(cpw)), "gq_gemv_plan")
    return r.value, ks.value, cpw.value


def gemv_workspace_bytes(fmt: int, k: int, batch: int) -> int:
    return load().gq_gemv_workspace_bytes(fmt, k, batch)


def gemv(fmt: int, d_packed, x, n: int, k: int, y=None, workspace: Workspace | None = None, stream=None):
    """y[b][n] = sum_k x[b][k] * W[n][k]; x float32 [batch][k] on the device."""
    import torch
    _require_device(d_packed, x)
    batch = 1 if x.dim() == 1 else x.shape[0]
    if y is None:
        y = torch.empty((batch, n), dtype=torch.float32, device=x.device)
    ws_ptr, ws_n = None, 0
    if workspace is not None:
        need = gemv_workspace_bytes(fmt, k, batch)
        buf = workspace.ensure(need)
        ws_ptr, ws_n = _ptr(buf), buf.numel()
    check(load().gq_gemv(fmt, _ptr(d_packed), _ptr(x), _ptr(y), n, k, batch, ws_ptr, ws_n, _stream(stream)),
          "gq_gemv")
    return y


def gemm_workspace_bytes(fmt: int, m: int, k: int) -> int:
    return load().gq_gemm_workspace_bytes(fmt, m, k)


def gemm(fmt: int, d_packed, a, n: int, k: int, out_dtype=None, c=None, workspace: Workspace | None = None,
         stream=None):
    """C[m][n] = sum_k A[m][k] * W[n][k]; A bf16/f16/f32 [m][k]; C f32 or bf16."""
    import torch
    _require_device(d_packed, a)
    dt = {torch.bfloat16: DT_BF16, torch.float16: DT_F16, torch.float32: DT_F32}[a.dtype]
    m = a.shape[0]
    out_dtype = out_dtype or torch.float32
    cdt = {torch.float32: DT_F32, torch.bfloat16: DT_BF16}[out_dtype]
    if c is None:
        c = torch.empty((m, n), dtype=out_dtype, device=a.device)
    ws_ptr, ws_n = None, 0
    if workspace is not None:
        buf = workspace.ensure(gemm_workspace_bytes(fmt, m, k))
        ws_ptr, ws_n = _ptr(buf), buf.numel()
    check(load().gq_gemm(fmt, _ptr(d_packed), _ptr(a), dt, _ptr(c), cdt, m, n, k, ws_ptr, ws_n, _stream(stream)),
          "gq_gemm")
    return c


def quantize_act_q8(a, stream=None):
    import torch
    _require_device(a)
    dt = {torch.bfloat16: DT_BF16, torch.float16: DT_F16, torch.float32: DT_F32}[a.dtype]
    m, k = a.shape
    q = torch.empty((m, k), dtype=torch.int8, device=a.device)
    d = torch.empty((m, k // 32), dtype=torch.float32, device=a.device)
    check(load().gq_quantize_act_q8(_ptr(a), dt, m, k, _ptr(q), _ptr(d), _stream(stream)), "gq_quantize_act_q8")
    return q, d


def gemm_q8_i8(d_packed, qa, da, n: int, c=None, stream=None):
    import torch
    _require_device(d_packed, qa, da)
    m, k = qa.shape
    if c is None:
        c = torch.empty((m, n), dtype=torch.float32, device=qa.device)
    check(load().gq_gemm_q8_i8(_ptr(d_packed), _ptr(qa), _ptr(da), _ptr(c), m, n, k, _stream(stream)),
          "gq_gemm_q8_i8")
    return c


def matmul(fmt: int, d_packed, a, n: int, k: int, c=None, stream=None):
    import torch
    _require_device(d_packed, a)
    m = a.shape[0]
    if c is None:
        c = torch.empty((m, n), dtype=torch.float32, device=a.device)
    check(load().gq_matmul(fmt, _ptr(d_packed), _ptr(a), _ptr(c), m, n, k, _stream(stream)), "gq_matmul")
    return c


def launch_int8_wt(a, b, scales, m, n, k, group_size=32, c=None, stream=None):
    """Reference-format INT8 weight-only matmul (gemm_kernels.hpp:43-47)."""
    import torch
    if c is None:
        c = torch.empty((m, n), dtype=torch.float32, device=a.device)
    check(load().gq_launch_gemm_mfma_int8_wt_fp32_acc32(_stream(stream), _ptr(a), _ptr(b), _ptr(c), _ptr(scales),
                                                         m, n, k, k, n, n, group_size),
          "gq_launch_gemm_mfma_int8_wt_fp32_acc32")
    return c


def launch_int4_wt(a, b, scales, head_scales, m, n, k, group_size=32, head_dim=0, force_gemv=False, c=None,
                   stream=None):
    """Reference-format INT4 weight-only matmul (gemm_kernels.hpp:49-57)."""
    import torch
    if c is None:
        c = torch.empty((m, n), dtype=torch.float32, device=a.device)
    check(load().gq_launch_gemm_mfma_int4_wt_fp32_acc32(
        _stream(stream), _ptr(a), _ptr(b), _ptr(c), _ptr(scales), _ptr(head_scales), m, n, k, k, n, n, group_size,
        head_dim, int(a.dtype == torch.float16), int(force_gemv)), "gq_launch_gemm_mfma_int4_wt_fp32_acc32")
    return c


def gemv_prep(fmt: int, x, k: int, workspace: Workspace, stream=None):
    """Prepare x [batch][k] once into `workspace` for several gemv_prepped calls."""
    _require_device(x)
    batch = 1 if x.dim() == 1 else x.shape[0]
    buf = workspace.ensure(gemv_workspace_bytes(fmt, k, batch))
    check(load().gq_gemv_prep(fmt, _ptr(x), k, batch, _ptr(buf), buf.numel(), _stream(stream)), "gq_gemv_prep")
    return batch


def gemv_prepped(fmt: int, d_packed, workspace: Workspace, y, n: int, k: int, batch: int, stream=None):
    _require_device(d_packed, y)
    check(load().gq_gemv_prepped(fmt, _ptr(d_packed), _ptr(workspace.buf), _ptr(y), n, k, batch, _stream(stream)),
          "gq_gemv_prepped")
    return y
