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
FMT_F16 = 1    # gq_dequant_gguf only
FMT_Q6_K = 14  # repack / dequant / gemv (no gemm)
FMT_Q6_K_GGML = 114
FORMATS = {"q4_0": FMT_Q4_0, "q8_0": FMT_Q8_0, "q4_k": FMT_Q4_K, "q4_k_ggml": FMT_Q4_K_GGML, "q6_k": FMT_Q6_K,
           "q6_k_ggml": FMT_Q6_K_GGML}

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
    "gq_repack_rows": (ctypes.c_int, [ctypes.c_int, _vp, _c_size, _c_size, _c_size, _c_size, _vp, _vp]),
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
    "gq_gemv_multi": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, _vp, _vp, _c_size, _vp, _vp, ctypes.c_int, _vp,
                                     ctypes.c_float, _vp]),
    "gq_gemv_multi_plan": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, _vp, _c_size, ctypes.c_int,
                                          ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int),
                                          ctypes.POINTER(ctypes.c_int)]),
    "gq_gemv_swiglu": (ctypes.c_int, [ctypes.c_int, _vp, _vp, _c_size, _c_size, _vp, _vp, ctypes.c_int, _vp,
                                      ctypes.c_float, _vp]),
    "gq_gemv_swiglu_plan": (ctypes.c_int, [ctypes.c_int, _c_size, _c_size, ctypes.c_int,
                                           ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]),
    "gq_convert_f32_to_f16": (ctypes.c_int, [_vp, _c_size, _vp, _vp]),
    "gq_transpose_kv": (ctypes.c_int, [ctypes.c_int, _vp, _c_size, _c_size, _vp, _vp]),
    "gq_requant_int8": (ctypes.c_int, [_vp, _c_size, _vp, _vp, _vp]),
    "gq_requant_int4": (ctypes.c_int, [_vp, _c_size, _vp, _vp, _vp]),
    "gq_head_scales": (ctypes.c_int, [_vp, _c_size, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, _vp, _vp]),
    "gq_split_q8_0": (ctypes.c_int, [_vp, _c_size, _vp, _vp, _vp]),
    "gq_gemm_static_max_bytes": (_c_size, []),
    "gq_gemm_static": (ctypes.c_int, [ctypes.c_int, _vp, _vp, ctypes.c_int, _vp, ctypes.c_int, _c_size, _c_size,
                                      _c_size, _vp]),
    "gq_gemm_f16w": (ctypes.c_int, [_vp, _vp, _vp, _c_size, _c_size, _c_size, _vp]),
    "gq_launch_gemm_mixed_f16f32": (ctypes.c_int, [_vp, _vp, _vp, _vp] + [ctypes.c_uint32] * 6),
    "gq_launch_gemm_mfma_mixed_f16f32": (ctypes.c_int, [_vp, _vp, _vp, _vp] + [ctypes.c_uint32] * 6),
    "gq_launch_gemm_mfma_int8_wt_fp32_acc32": (
        ctypes.c_int, [_vp, _vp, _vp, _vp, _vp] + [ctypes.c_uint32] * 7),
    "gq_launch_gemm_mfma_int4_wt_fp32_acc32": (
        ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp] + [ctypes.c_uint32] * 8 + [ctypes.c_int, ctypes.c_int]),
}

# include/gq_gguf.h
_SIGS_GGUF = {
    "gq_gguf_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "gq_gguf_open_error": (ctypes.c_char_p, []),
    "gq_gguf_close": (None, [_vp]),
    "gq_gguf_error": (ctypes.c_char_p, [_vp]),
    "gq_gguf_tensor_count": (_c_size, [_vp]),
    "gq_gguf_tensor_info": (ctypes.c_int, [_vp, _c_size, _vp]),
    "gq_gguf_find": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.POINTER(_c_size)]),
    "gq_gguf_get_config": (ctypes.c_int, [_vp, _vp]),
    "gq_gguf_vocab_token": (ctypes.c_int, [_vp, _c_size, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_c_size)]),
    "gq_gguf_set_q4k_layout": (ctypes.c_int, [_vp, ctypes.c_int]),
    "gq_gguf_read_raw": (ctypes.c_int, [_vp, ctypes.c_char_p, _vp, _c_size]),
    "gq_gguf_plan_load": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.c_int, _vp]),
    "gq_gguf_load": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.c_int, _vp, _c_size, _vp, _c_size, _vp, _c_size]),
    "gq_gguf_load_quant_many": (ctypes.c_int, [_vp, _c_size, _vp, _vp, _vp]),
    # include/gq_greta.h
    "gq_greta_write": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(_c_size)]),
    "gq_greta_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "gq_greta_open_error": (ctypes.c_char_p, []),
    "gq_greta_close": (None, [_vp]),
    "gq_greta_error": (ctypes.c_char_p, [_vp]),
    "gq_greta_tensor_count": (_c_size, [_vp]),
    "gq_greta_tensor_info": (ctypes.c_int, [_vp, _c_size, _vp]),
    "gq_greta_find": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.POINTER(_c_size)]),
    "gq_greta_get_config": (ctypes.c_int, [_vp, _vp]),
    "gq_greta_load": (ctypes.c_int, [_vp, ctypes.c_char_p, _vp, _c_size, _vp, _c_size, _vp, _c_size]),
}
_SIGS.update(_SIGS_GGUF)


class ChainOp(ctypes.Structure):
    """gq_chain_op (include/gq_chain.h)."""
    _fields_ = [("w", _vp), ("w_up", _vp), ("x", _vp), ("gamma", _vp), ("resid", _vp), ("y", _vp),
                ("N", ctypes.c_uint32), ("K", ctypes.c_uint32), ("k_offset", ctypes.c_uint32),
                ("k_total", ctypes.c_uint32), ("x_head_dim", ctypes.c_uint32), ("x_group", ctypes.c_uint32),
                ("dep", ctypes.c_int32 * 3)]


# include/gq_chain.h
_SIGS.update({
    "gq_gemv_chain_workspace_bytes": (ctypes.c_int, [ctypes.c_int, _vp, ctypes.c_int, ctypes.POINTER(_c_size)]),
    "gq_gemv_chain_plan": (ctypes.c_int, [ctypes.c_int, _vp, ctypes.c_int, ctypes.c_float, _vp, _c_size]),
    "gq_gemv_chain_run": (ctypes.c_int, [_vp, _vp]),
    "gq_gemv_chain_error": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_int)]),
})

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
    # PyTorch's HIP runtime must be loaded before libgq's (same soname): with
    # the order reversed, libgq's HIP calls report no device on this image
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
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


def repack_rows(fmt: int, d_gguf_rows, n: int, k: int, row0: int, rows: int, d_packed, stream=None):
    """Repacks GGUF rows [row0, row0 + rows) into the whole tensor's T16 buffer."""
    _require_device(d_gguf_rows)
    _require_device(d_packed)
    check(load().gq_repack_rows(fmt, _ptr(d_gguf_rows), n, k, row0, rows, _ptr(d_packed), _stream(stream)),
          "gq_repack_rows")


def dequant_gguf(fmt: int, d_blocks, n_blocks: int, stream=None):
    import torch
    _require_device(d_blocks)
    per = 256 if fmt in (FMT_Q4_K, FMT_Q4_K_GGML, FMT_Q6_K, FMT_Q6_K_GGML) else (1 if fmt == FMT_F16 else 32)
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


def gemm_f16w(w, a, n: int, k: int, c=None, stream=None):
    """C[m][n] = sum_k A[m][k] * W[n][k]: fp16 weights W [n][k] (row-major,
    as GGUF F16 tensors), A float32 [m][k], C float32 (gq_gemm_f16w)."""
    import torch
    _require_device(w, a)
    m = 1 if a.dim() == 1 else a.shape[0]
    if c is None:
        c = torch.empty((m, n), dtype=torch.float32, device=a.device)
    check(load().gq_gemm_f16w(_ptr(w), _ptr(a), _ptr(c), m, n, k, _stream(stream)), "gq_gemm_f16w")
    return c


def launch_mixed_f16f32(a, w, m, n, k, mfma=False, c=None, stream=None):
    """The reference's FP16-weight launchers (gemm_kernels.hpp:30-44)."""
    import torch
    if c is None:
        c = torch.empty((m, n), dtype=torch.float32, device=a.device)
    f = load().gq_launch_gemm_mfma_mixed_f16f32 if mfma else load().gq_launch_gemm_mixed_f16f32
    check(f(_stream(stream), _ptr(a), _ptr(w), _ptr(c), m, n, k, k, n, n), "gq_launch_gemm_mixed_f16f32")
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


def _chain_ops(ops):
    arr = (ChainOp * len(ops))()
    for i, o in enumerate(ops):
        a = arr[i]
        adr = lambda t: t.data_ptr() if t is not None else None  # noqa: E731
        a.w, a.w_up = adr(o["w"]), adr(o.get("w_up"))
        a.x, a.gamma, a.resid, a.y = adr(o["x"]), adr(o.get("gamma")), adr(o.get("resid")), adr(o["y"])
        a.N, a.K = o["N"], o["K"]
        a.k_offset, a.k_total = o.get("k_offset", 0), o.get("k_total", 0)
        a.x_head_dim, a.x_group = o.get("x_head_dim", 0), o.get("x_group", 0)
        deps = list(o.get("deps", [])) + [-1] * 3
        for q in range(3):
            a.dep[q] = deps[q]
    return arr


def chain_workspace_bytes(fmt: int, ops) -> int:
    """Workspace bytes of a chain plan (host only).  ops: dicts with keys w,
    x, y, N, K and optionally w_up, gamma, resid, k_offset, k_total,
    x_head_dim, x_group, deps (see include/gq_chain.h)."""
    arr = _chain_ops(ops)
    n = _c_size(0)
    check(load().gq_gemv_chain_workspace_bytes(fmt, ctypes.cast(arr, _vp), len(ops), ctypes.byref(n)),
          "gq_gemv_chain_workspace_bytes")
    return n.value


class Chain:
    """A planned chain of decode GEMVs (gq_gemv_chain_plan); run() launches it."""

    def __init__(self, fmt: int, ops, device, eps: float = 1e-5):
        import torch
        self.ops = ops  # (keeps the tensors alive)
        arr = _chain_ops(ops)
        nbytes = chain_workspace_bytes(fmt, ops)
        self.ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
        check(load().gq_gemv_chain_plan(fmt, ctypes.cast(arr, _vp), len(ops), eps, _ptr(self.ws), nbytes),
              "gq_gemv_chain_plan")

    def run(self, stream=None):
        check(load().gq_gemv_chain_run(_ptr(self.ws), _stream(stream)), "gq_gemv_chain_run")

    def error(self) -> int:
        e = ctypes.c_int(0)
        check(load().gq_gemv_chain_error(_ptr(self.ws), ctypes.byref(e)), "gq_gemv_chain_error")
        return e.value


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


# ---- fused decode GEMVs ----------------------------------------------------------
def gemv_multi(fmt: int, mats, x, k: int, gamma=None, eps: float = 1e-5, ys=None, stream=None):
    """mats: list of (d_packed, n).  Returns [y_i [batch][n_i]] (one launch)."""
    import torch
    _require_device(x)
    batch = 1 if x.dim() == 1 else x.shape[0]
    if ys is None:
        ys = [torch.empty((batch, n), dtype=torch.float32, device=x.device) for _, n in mats]
    P = (_vp * len(mats))(*[t.data_ptr() for t, _ in mats])
    Y = (_vp * len(mats))(*[t.data_ptr() for t in ys])
    N = (_c_size * len(mats))(*[n for _, n in mats])
    check(load().gq_gemv_multi(fmt, len(mats), ctypes.cast(P, _vp), ctypes.cast(N, _vp), k, _ptr(x),
                               ctypes.cast(Y, _vp), batch, _ptr(gamma), eps, _stream(stream)), "gq_gemv_multi")
    return ys


def gemv_multi_plan(fmt: int, ns, k: int, batch: int):
    N = (_c_size * len(ns))(*ns)
    r, ks, cpw = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    check(load().gq_gemv_multi_plan(fmt, len(ns), ctypes.cast(N, _vp), k, batch, ctypes.byref(r), ctypes.byref(ks),
                                    ctypes.byref(cpw)), "gq_gemv_multi_plan")
    return r.value, ks.value, cpw.value


def gemv_swiglu(fmt: int, gate, up, x, n: int, k: int, gamma=None, eps: float = 1e-5, y=None, stream=None):
    import torch
    _require_device(gate, up, x)
    batch = 1 if x.dim() == 1 else x.shape[0]
    if y is None:
        y = torch.empty((batch, n), dtype=torch.float32, device=x.device)
    check(load().gq_gemv_swiglu(fmt, _ptr(gate), _ptr(up), n, k, _ptr(x), _ptr(y), batch, _ptr(gamma), eps,
                                _stream(stream)), "gq_gemv_swiglu")
    return y


def gemv_swiglu_plan(fmt: int, n: int, k: int, batch: int):
    ks, cpw = ctypes.c_int(), ctypes.c_int()
    check(load().gq_gemv_swiglu_plan(fmt, n, k, batch, ctypes.byref(ks), ctypes.byref(cpw)), "gq_gemv_swiglu_plan")
    return ks.value, cpw.value


# ---- load-time conversions (bit-exact with the reference loader) ------------
def convert_f32_to_f16(w, stream=None):
    """Reference truncating fp32 -> fp16 (weight_loader.cpp:112-123); returns int16 bits."""
    import torch
    _require_device(w)
    out = torch.empty(w.numel(), dtype=torch.int16, device=w.device)
    check(load().gq_convert_f32_to_f16(_ptr(w), w.numel(), _ptr(out), _stream(stream)), "gq_convert_f32_to_f16")
    return out


def transpose_kv(t, model_dim: int, kv_dim: int, stream=None):
    import torch
    _require_device(t)
    out = torch.empty(t.numel(), dtype=t.dtype, device=t.device)
    check(load().gq_transpose_kv(t.element_size(), _ptr(t), model_dim, kv_dim, _ptr(out), _stream(stream)),
          "gq_transpose_kv")
    return out


def requant_int8(w, stream=None):
    import torch
    _require_device(w)
    n = w.numel()
    q = torch.empty(n, dtype=torch.int8, device=w.device)
    s = torch.empty((n + 31) // 32, dtype=torch.float32, device=w.device)
    check(load().gq_requant_int8(_ptr(w), n, _ptr(q), _ptr(s), _stream(stream)), "gq_requant_int8")
    return q, s


def requant_int4(w, stream=None):
    import torch
    _require_device(w)
    n = w.numel()
    q = torch.empty((n + 1) // 2, dtype=torch.uint8, device=w.device)
    s = torch.empty((n + 31) // 32, dtype=torch.float32, device=w.device)
    check(load().gq_requant_int4(_ptr(w), n, _ptr(q), _ptr(s), _stream(stream)), "gq_requant_int4")
    return q, s


def head_scales(w, num_heads: int, head_dim: int, dim: int, stream=None):
    import torch
    _require_device(w)
    out = torch.empty(num_heads, dtype=torch.float32, device=w.device)
    check(load().gq_head_scales(_ptr(w), w.numel(), num_heads, head_dim, dim, _ptr(out), _stream(stream)),
          "gq_head_scales")
    return out


def split_q8_0(d_blocks, n_blocks: int, stream=None):
    import torch
    _require_device(d_blocks)
    q = torch.empty(n_blocks * 32, dtype=torch.int8, device=d_blocks.device)
    s = torch.empty(n_blocks, dtype=torch.float32, device=d_blocks.device)
    check(load().gq_split_q8_0(_ptr(d_blocks), n_blocks, _ptr(q), _ptr(s), _stream(stream)), "gq_split_q8_0")
    return q, s


# ---- GGUF loader (include/gq_gguf.h) ----------------------------------------
LOAD_F32, LOAD_F16, LOAD_INT8, LOAD_INT4, LOAD_QUANT = range(5)


class _Tensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 256), ("dtype", ctypes.c_char * 16), ("ggml_type", ctypes.c_uint32),
                ("n_dims", ctypes.c_uint32), ("shape", ctypes.c_uint64 * 8), ("offset", ctypes.c_uint64),
                ("size_bytes", ctypes.c_uint64)]


class _Config(ctypes.Structure):
    _fields_ = [(f, ctypes.c_uint32) for f in ("dim", "num_heads", "num_heads_kv", "num_layers", "vocab_size",
                                                "hidden_dim", "head_dim", "max_seq_len")] + \
               [("rope_base", ctypes.c_float), ("rms_eps", ctypes.c_float)]


class _Plan(ctypes.Structure):
    _fields_ = [("n_elem", ctypes.c_uint64), ("bytes", ctypes.c_uint64), ("scale_bytes", ctypes.c_uint64),
                ("num_heads", ctypes.c_uint32), ("has_head_scales", ctypes.c_int32), ("is_qkv", ctypes.c_int32),
                ("transpose", ctypes.c_int32), ("fmt", ctypes.c_int32), ("N", ctypes.c_uint64),
                ("K", ctypes.c_uint64)]


class GGUF:
    """GGUF file opened through libgq's loader (GGUFLoader, weight_loader.cpp:467-1008).

    Parsing needs no GPU; load() converts on the GPU into torch device tensors.
    """

    def __init__(self, path: str):
        lib = load()
        h = _vp()
        st = lib.gq_gguf_open(os.fsencode(path), ctypes.byref(h))
        if st != 0:
            raise GQError(f"gq_gguf_open({path}) failed: {lib.gq_gguf_open_error().decode()}")
        self._h = h
        self.path = path

    def close(self):
        if self._h:
            load().gq_gguf_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _check(self, st, what):
        if st != 0:
            raise GQError(f"{what} failed ({st}): {load().gq_gguf_error(self._h).decode()}")

    def tensors(self):
        lib = load()
        out = []
        for i in range(lib.gq_gguf_tensor_count(self._h)):
            t = _Tensor()
            self._check(lib.gq_gguf_tensor_info(self._h, i, ctypes.byref(t)), "gq_gguf_tensor_info")
            out.append({"name": t.name.decode(), "dtype": t.dtype.decode(), "ggml_type": t.ggml_type,
                        "shape": [int(t.shape[d]) for d in range(t.n_dims)], "offset": int(t.offset),
                        "size_bytes": int(t.size_bytes)})
        return out

    def config(self):
        c = _Config()
        self._check(load().gq_gguf_get_config(self._h, ctypes.byref(c)), "gq_gguf_get_config")
        return {f: getattr(c, f) for f, _ in _Config._fields_}

    def vocab(self):
        lib = load()
        n = self.config()["vocab_size"]
        out = []
        for i in range(n):
            s, ln = ctypes.c_char_p(), _c_size()
            if lib.gq_gguf_vocab_token(self._h, i, ctypes.byref(s), ctypes.byref(ln)) != 0:
                break
            out.append(ctypes.string_at(s, ln.value))
        return out

    def set_q4k_layout(self, ggml: bool):
        self._check(load().gq_gguf_set_q4k_layout(self._h, int(ggml)), "gq_gguf_set_q4k_layout")

    def read_raw(self, name: str):
        import numpy as np
        t = next(t for t in self.tensors() if t["name"] == name)
        out = np.empty(t["size_bytes"], dtype=np.uint8)
        self._check(load().gq_gguf_read_raw(self._h, name.encode(), out.ctypes.data, out.size), "gq_gguf_read_raw")
        return out

    def plan(self, name: str, kind: int):
        p = _Plan()
        self._check(load().gq_gguf_plan_load(self._h, name.encode(), kind, ctypes.byref(p)), "gq_gguf_plan_load")
        return {f: getattr(p, f) for f, _ in _Plan._fields_}

    def load_quant_many(self, names, outs):
        """GQ_LOAD_QUANT of every name into the matching device tensor of `outs`
        (uint8, at least the planned bytes) in one pipelined pass."""
        n = len(names)
        if n != len(outs):
            raise ValueError("names and outs differ in length")
        _require_device(*outs)
        enc = [nm.encode() for nm in names]
        N = (ctypes.c_char_p * n)(*enc)
        P = (_vp * n)(*[t.data_ptr() for t in outs])
        B = (_c_size * n)(*[t.numel() * t.element_size() for t in outs])
        self._check(load().gq_gguf_load_quant_many(self._h, n, ctypes.cast(N, _vp), ctypes.cast(P, _vp),
                                                   ctypes.cast(B, _vp)), "gq_gguf_load_quant_many")

    def load(self, name: str, kind: int, device="cuda"):
        """Returns (data, scales, head_scales, plan) as device tensors (None where absent)."""
        import torch
        p = self.plan(name, kind)
        out = torch.empty(max(p["bytes"], 1), dtype=torch.uint8, device=device)
        sc = torch.empty(max(p["scale_bytes"], 1), dtype=torch.uint8, device=device) if p["scale_bytes"] else None
        hs = torch.empty(p["num_heads"], dtype=torch.float32, device=device) if p["has_head_scales"] else None
        self._check(load().gq_gguf_load(self._h, name.encode(), kind, _ptr(out), out.numel(), _ptr(sc),
                                        sc.numel() if sc is not None else 0, _ptr(hs),
                                        hs.numel() * 4 if hs is not None else 0), "gq_gguf_load")
        out = out[:p["bytes"]]
        if kind == LOAD_F32:
            out = out.view(torch.float32)
        elif kind == LOAD_F16:
            out = out.view(torch.int16)
        elif kind == LOAD_INT8:
            out = out.view(torch.int8)
        if sc is not None:
            sc = sc[:p["scale_bytes"]].view(torch.float32)
        return out, sc, hs, p


# ---- .greta files (include/gq_greta.h) ---------------------------------------
GRETA_INT4, GRETA_Q4_K, GRETA_Q4_0, GRETA_Q8_0, GRETA_Q4_K_GGML, GRETA_Q6_K, GRETA_Q6_K_GGML = 4, 5, 8, 9, 10, 11, 12


class _GretaTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 256), ("dtype", ctypes.c_uint32), ("n_dims", ctypes.c_uint32),
                ("shape", ctypes.c_uint64 * 8), ("group_size", ctypes.c_uint32), ("num_heads", ctypes.c_uint32),
                ("w_bytes", ctypes.c_uint64), ("s_bytes", ctypes.c_uint64), ("h_bytes", ctypes.c_uint64),
                ("fmt", ctypes.c_int32), ("N", ctypes.c_uint64), ("K", ctypes.c_uint64)]


def greta_write(gguf: "GGUF", path: str, kind: int = LOAD_QUANT) -> int:
    """Writes a .greta file from an open GGUF: kind LOAD_QUANT (T16 records,
    host repack) or LOAD_INT4 (the reference tool's INT4 records, on the GPU).
    Returns the record count."""
    n = _c_size(0)
    gguf._check(load().gq_greta_write(gguf._h, os.fsencode(path), kind, ctypes.byref(n)), "gq_greta_write")
    return n.value


class Greta:
    """.greta file opened through libgq's reader (GretaLoader)."""

    def __init__(self, path: str):
        lib = load()
        h = _vp()
        if lib.gq_greta_open(os.fsencode(path), ctypes.byref(h)) != 0:
            raise GQError(f"gq_greta_open({path}) failed: {lib.gq_greta_open_error().decode()}")
        self._h = h

    def close(self):
        if self._h:
            load().gq_greta_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _check(self, st, what):
        if st != 0:
            raise GQError(f"{what} failed ({st}): {load().gq_greta_error(self._h).decode()}")

    def tensors(self):
        lib = load()
        out = []
        for i in range(lib.gq_greta_tensor_count(self._h)):
            t = _GretaTensor()
            self._check(lib.gq_greta_tensor_info(self._h, i, ctypes.byref(t)), "gq_greta_tensor_info")
            out.append({"name": t.name.decode(), "dtype": t.dtype, "shape": [int(t.shape[d]) for d in range(t.n_dims)],
                        "group_size": t.group_size, "num_heads": t.num_heads, "w_bytes": int(t.w_bytes),
                        "s_bytes": int(t.s_bytes), "h_bytes": int(t.h_bytes), "fmt": t.fmt, "N": int(t.N),
                        "K": int(t.K)})
        return out

    def config(self):
        c = _Config()
        self._check(load().gq_greta_get_config(self._h, ctypes.byref(c)), "gq_greta_get_config")
        return {f: getattr(c, f) for f, _ in _Config._fields_}

    def load(self, name: str, device="cuda"):
        """Returns (w, s, h) uint8 device tensors (None where the record has none)."""
        import torch
        t = next(t for t in self.tensors() if t["name"] == name)
        w = torch.empty(max(t["w_bytes"], 1), dtype=torch.uint8, device=device)
        s = torch.empty(t["s_bytes"], dtype=torch.uint8, device=device) if t["s_bytes"] else None
        h = torch.empty(t["h_bytes"], dtype=torch.uint8, device=device) if t["h_bytes"] else None
        self._check(load().gq_greta_load(self._h, name.encode(), _ptr(w), w.numel(), _ptr(s),
                                         s.numel() if s is not None else 0, _ptr(h),
                                         h.numel() if h is not None else 0), "gq_greta_load")
        return w[:t["w_bytes"]], s, h

