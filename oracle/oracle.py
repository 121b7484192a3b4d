"""Python access to the CPU oracle (oracle/gq_oracle.c) and to the reference's
own CPU functions compiled into oracle/_ref/libgqref.so.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, always as the checker / baseline, never as the
thing measured or shipped.

Also holds the seeded synthetic GGUF generators for the benchmark configurations:
  Q8_0: q ~ U[-127,127], d = fp16(|N(0,1)| * 0.02)
  Q4_0: nibbles ~ U[0,15], d = fp16(|N(0,1)| * 0.02)
  Q4_K: 12 code bytes ~ U[0,255] (codes U[0,63]), nibbles ~ U[0,15],
        d, dmin = fp16(|N(0,1)| * 0.01)
fp16 conversion is round-to-nearest-even (numpy), the same rounding as
CpuReference::float_to_half (cpu_reference.hpp:19-38) for normal values.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "_build", "libgqoracle.so")
REF_SO = os.path.join(HERE, "_ref", "libgqref.so")

Q4_0, Q8_0, Q4_K, Q6_K, Q4_K_GGML, Q6_K_GGML = 2, 8, 12, 14, 112, 114
BLOCK_ELEMS = {Q4_0: 32, Q8_0: 32, Q4_K: 256, Q4_K_GGML: 256, Q6_K: 256, Q6_K_GGML: 256}
BLOCK_BYTES = {Q4_0: 18, Q8_0: 34, Q4_K: 144, Q4_K_GGML: 144, Q6_K: 210, Q6_K_GGML: 210}

_lib = None
_ref = None
_F = ctypes.POINTER(ctypes.c_float)


def build():
    """Compile the oracle (and the reference harness where the tree exists)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            build()
        L = ctypes.CDLL(ORACLE_SO)
        vp, sz, i = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
        L.gqo_fp16_to_fp32_n.argtypes = [vp, sz, vp]
        L.gqo_rmsnorm.argtypes = [vp, vp, i, i, ctypes.c_float, vp]
        L.gqo_swiglu.argtypes = [vp, vp, sz, vp]
        L.gqo_fp32_to_fp16_trunc_n.argtypes = [vp, sz, vp]
        L.gqo_fp16_to_fp32.restype = ctypes.c_float
        L.gqo_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.gqo_float_to_half.restype = ctypes.c_uint16
        L.gqo_float_to_half.argtypes = [ctypes.c_float]
        L.gqo_dequant.argtypes = [i, vp, sz, vp]
        L.gqo_gemv.argtypes = [i, vp, vp, vp, i, i, i, i]
        L.gqo_gemm.argtypes = [i, vp, vp, vp, i, i, i, i]
        L.gqo_gemm_ref.argtypes = [vp, vp, vp, i, i, i]
        L.gqo_requant_int8.argtypes = [vp, sz, vp, vp]
        L.gqo_requant_int4.argtypes = [vp, sz, vp, vp]
        L.gqo_head_scales.argtypes = [vp, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, vp]
        L.gqo_gqa_transpose.argtypes = [vp, ctypes.c_uint32, ctypes.c_uint32, vp]
        L.gqo_gemm_int8_wt.argtypes = [vp, vp, vp, vp, i, i, i, i, i]
        L.gqo_gemm_int4_wt.argtypes = [vp, vp, vp, vp, vp, i, i, i, i, i, i]
        L.gqo_quantize_act_q8.argtypes = [vp, i, i, vp, vp]
        L.gqo_gemm_q8_i8.argtypes = [vp, vp, vp, vp, i, i, i, i]
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_SO)


def ref():
    """The reference's own CPU functions (oracle/_ref), or None if not built."""
    global _ref
    if _ref is None and ref_available():
        # the reference's loader is HIP code: PyTorch's HIP runtime (same
        # soname) must be loaded first, or the two runtimes disagree and the
        # reference's allocations report no device once torch holds the GPU
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        R = ctypes.CDLL(REF_SO)
        vp, sz, i = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
        R.gqref_fp16_to_fp32.restype = ctypes.c_float
        R.gqref_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        R.gqref_fp32_to_fp16.restype = ctypes.c_uint16
        R.gqref_fp32_to_fp16.argtypes = [ctypes.c_float]
        R.gqref_half_to_float.restype = ctypes.c_float
        R.gqref_half_to_float.argtypes = [ctypes.c_uint16]
        R.gqref_float_to_half.restype = ctypes.c_uint16
        R.gqref_float_to_half.argtypes = [ctypes.c_float]
        R.gqref_dequant_q4_k.argtypes = [vp, sz, vp]
        R.gqref_dequant_q6_k.argtypes = [vp, sz, vp]
        R.gqref_gemm.argtypes = [vp, vp, vp, i, i, i]
        R.gqref_gguf_parse.argtypes = [ctypes.c_char_p, vp, i, vp, ctypes.c_char_p, i]
        R.gqref_gguf_parse.restype = i
        u64p = ctypes.POINTER(ctypes.c_uint64)
        R.gqref_gguf_load.argtypes = [ctypes.c_char_p, ctypes.c_char_p, i, vp, ctypes.c_uint64, u64p, vp,
                                      ctypes.c_uint64, u64p, vp, ctypes.c_uint64, u64p, ctypes.c_char_p, i]
        R.gqref_gguf_load.restype = i
        _ref = R
    return _ref


def _p(a):
    return ctypes.c_void_p(a.ctypes.data)


# ---- oracle functions ------------------------------------------------------
def fp16_to_fp32(h) -> np.ndarray:
    """Reference fp16 -> fp32 (NaN -> Inf) of a uint16 array."""
    h = np.ascontiguousarray(h, dtype=np.uint16).ravel()
    out = np.empty(h.size, dtype=np.float32)
    lib().gqo_fp16_to_fp32_n(_p(h), h.size, _p(out))
    return out


def rmsnorm(x, gamma, eps):
    """fp64 RMS normalisation of each row of x (rows x K) times gamma."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    x2 = x.reshape(-1, x.shape[-1])
    gamma = np.ascontiguousarray(gamma, dtype=np.float32)
    out = np.empty(x2.shape, dtype=np.float64)
    lib().gqo_rmsnorm(_p(x2), _p(gamma), x2.shape[0], x2.shape[1], float(eps), _p(out))
    return out.reshape(x.shape)


def swiglu(g, u):
    g = np.ascontiguousarray(g, dtype=np.float64)
    u = np.ascontiguousarray(u, dtype=np.float64)
    out = np.empty(g.shape, dtype=np.float64)
    lib().gqo_swiglu(_p(g), _p(u), g.size, _p(out))
    return out


def fp32_to_fp16_trunc(f) -> np.ndarray:
    """Reference truncating fp32 -> fp16 bits of a float32 array."""
    f = np.ascontiguousarray(f, dtype=np.float32).ravel()
    out = np.empty(f.size, dtype=np.uint16)
    lib().gqo_fp32_to_fp16_trunc_n(_p(f), f.size, _p(out))
    return out


def dequant(fmt: int, blocks: np.ndarray) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8).ravel()
    nb = blocks.size // BLOCK_BYTES[fmt]
    out = np.empty(nb * BLOCK_ELEMS[fmt], dtype=np.float32)
    if lib().gqo_dequant(fmt, _p(blocks), nb, _p(out)) != 0:
        raise RuntimeError("gqo_dequant failed")
    return out


def gemv(fmt: int, w: np.ndarray, x: np.ndarray, n: int, k: int, threads: int = 0) -> np.ndarray:
    """y[b][n] (fp64 accumulation); x float32 [b][k]."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, k)
    y = np.empty((x.shape[0], n), dtype=np.float32)
    if lib().gqo_gemv(fmt, _p(w), _p(x), _p(y), n, k, x.shape[0], threads) != 0:
        raise RuntimeError("gqo_gemv failed")
    return y


def gemm_ref(A, B):
    A = np.ascontiguousarray(A, dtype=np.float32)
    B = np.ascontiguousarray(B, dtype=np.float32)
    M, K = A.shape
    N = B.shape[1]
    C = np.empty((M, N), dtype=np.float32)
    lib().gqo_gemm_ref(_p(A), _p(B), _p(C), M, N, K)
    return C


def requant_int8(w):
    w = np.ascontiguousarray(w, dtype=np.float32).ravel()
    q = np.empty(w.size, dtype=np.int8)
    s = np.empty((w.size + 31) // 32, dtype=np.float32)
    lib().gqo_requant_int8(_p(w), w.size, _p(q), _p(s))
    return q, s


def requant_int4(w):
    w = np.ascontiguousarray(w, dtype=np.float32).ravel()
    p = np.zeros((w.size + 1) // 2, dtype=np.uint8)
    s = np.empty((w.size + 31) // 32, dtype=np.float32)
    lib().gqo_requant_int4(_p(w), w.size, _p(p), _p(s))
    return p, s


def head_scales(w, num_heads, head_dim, dim):
    w = np.ascontiguousarray(w, dtype=np.float32)
    h = np.empty(num_heads, dtype=np.float32)
    lib().gqo_head_scales(_p(w), num_heads, head_dim, dim, _p(h))
    return h


def gqa_transpose(w, model_dim, kv_dim):
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty(model_dim * kv_dim, dtype=np.float32)
    lib().gqo_gqa_transpose(_p(w), model_dim, kv_dim, _p(out))
    return out


def _gemv_route(m, gemv_route):
    """The reference launchers take the GEMV kernels for M <= 32 (or
    force_gemv), the MFMA kernels above (gemm_kernels.hip:749, 917)."""
    return int(m <= 32 if gemv_route is None else gemv_route)


def gemm_int8_wt(x, q, s, m, n, k, gs=32, gemv_route=None):
    """Reference INT8 launcher math; the scale index follows the route the
    reference takes for m rows unless gemv_route is given."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.ascontiguousarray(q, dtype=np.int8)
    s = np.ascontiguousarray(s, dtype=np.float32)
    y = np.empty((m, n), dtype=np.float32)
    lib().gqo_gemm_int8_wt(_p(x), _p(q), _p(s), _p(y), m, n, k, gs, _gemv_route(m, gemv_route))
    return y


def gemm_int4_wt(x, packed, s, hs, m, n, k, gs=32, head_dim=0, gemv_route=None):
    """Reference INT4 launcher math (K even); scale index as gemm_int8_wt."""
    assert k % 2 == 0
    x = np.ascontiguousarray(x, dtype=np.float32)
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    s = np.ascontiguousarray(s, dtype=np.float32)
    y = np.empty((m, n), dtype=np.float32)
    hsp = _p(np.ascontiguousarray(hs, dtype=np.float32)) if hs is not None else None
    lib().gqo_gemm_int4_wt(_p(x), _p(packed), _p(s), hsp, _p(y), m, n, k, gs, head_dim, _gemv_route(m, gemv_route))
    return y


def quantize_act_q8(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    m, k = a.shape
    q = np.empty((m, k), dtype=np.int8)
    d = np.empty((m, k // 32), dtype=np.float32)
    lib().gqo_quantize_act_q8(_p(a), m, k, _p(q), _p(d))
    return q, d


def gemm_q8_i8(w, qa, da, n, threads=0):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    qa = np.ascontiguousarray(qa, dtype=np.int8)
    da = np.ascontiguousarray(da, dtype=np.float32)
    m, k = qa.shape
    c = np.empty((m, n), dtype=np.float32)
    lib().gqo_gemm_q8_i8(_p(w), _p(qa), _p(da), _p(c), m, n, k, threads)
    return c


# ---- synthetic GGUF tensors -------------------------------------------------
def _scales16(rng, n, mult):
    return (np.abs(rng.standard_normal(n)) * mult).astype(np.float32).astype(np.float16).view(np.uint16)


def gen_weights(fmt: int, n: int, k: int, seed: int) -> np.ndarray:
    """Seeded synthetic GGUF tensor (N rows of K elements), uint8 bytes."""
    rng = np.random.default_rng(seed)
    be, bb = BLOCK_ELEMS[fmt], BLOCK_BYTES[fmt]
    nb = n * (k // be)
    out = np.empty((nb, bb), dtype=np.uint8)
    if fmt == Q4_0:
        out[:, 0:2] = _scales16(rng, nb, 0.02).view(np.uint8).reshape(nb, 2)
        out[:, 2:] = rng.integers(0, 256, size=(nb, 16), dtype=np.uint8)
    elif fmt == Q8_0:
        out[:, 0:2] = _scales16(rng, nb, 0.02).view(np.uint8).reshape(nb, 2)
        out[:, 2:] = rng.integers(-127, 128, size=(nb, 32), dtype=np.int16).astype(np.int8).view(np.uint8)
    elif fmt in (Q4_K, Q4_K_GGML):
        out[:, 0:2] = _scales16(rng, nb, 0.01).view(np.uint8).reshape(nb, 2)
        out[:, 2:4] = _scales16(rng, nb, 0.01).view(np.uint8).reshape(nb, 2)
        out[:, 4:] = rng.integers(0, 256, size=(nb, 140), dtype=np.uint8)
    elif fmt in (Q6_K, Q6_K_GGML):
        out[:, :208] = rng.integers(0, 256, size=(nb, 208), dtype=np.uint8)
        out[:, 192:208] = rng.integers(-32, 32, size=(nb, 16), dtype=np.int8).view(np.uint8)
        out[:, 208:210] = _scales16(rng, nb, 0.01).view(np.uint8).reshape(nb, 2)
    else:
        raise ValueError(fmt)
    return out.reshape(-1)


def gen_x(batch: int, k: int, seed: int) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal((batch, k)).astype(np.float32)


def rel_l2(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


# ---- the reference's own GGUF loader (oracle/_ref) ---------------------------
class _RefTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 128), ("dtype", ctypes.c_char * 16), ("shape", ctypes.c_uint64 * 4),
                ("n_dims", ctypes.c_uint32), ("offset", ctypes.c_uint64), ("size_bytes", ctypes.c_uint64)]


class _RefConfig(ctypes.Structure):
    _fields_ = [(f, ctypes.c_uint32) for f in ("dim", "num_heads", "num_heads_kv", "num_layers", "vocab_size",
                                                "hidden_dim", "head_dim", "max_seq_len")] + \
               [("rope_base", ctypes.c_float), ("rms_eps", ctypes.c_float)]


def ref_gguf_parse(path: str, cap: int = 4096):
    """GGUFLoader::open + list_tensors + get_config of the reference, or
    (None, None, message) when it refuses the file."""
    R = ref()
    arr = (_RefTensor * cap)()
    cfg = _RefConfig()
    err = ctypes.create_string_buffer(512)
    n = R.gqref_gguf_parse(os.fsencode(path), ctypes.cast(arr, ctypes.c_void_p), cap, ctypes.byref(cfg), err, 512)
    if n < 0:
        return None, None, err.value.decode(errors="replace")
    ts = [{"name": t.name.decode(), "dtype": t.dtype.decode(), "shape": [int(t.shape[d]) for d in range(t.n_dims)],
           "offset": int(t.offset), "size_bytes": int(t.size_bytes)} for t in arr[:n]]
    return ts, {f: getattr(cfg, f) for f, _ in _RefConfig._fields_}, ""


def ref_gguf_load(path: str, name: str, kind: int, max_bytes: int):
    """The reference loader's load_tensor / _fp16 / _int8 / _int4 (kind 0..3),
    run on the GPU; returns (data bytes, scales f32, head scales f32)."""
    R = ref()
    out = np.empty(max_bytes, dtype=np.uint8)
    sc = np.empty(max_bytes // 8 + 64, dtype=np.float32)
    hs = np.empty(4096, dtype=np.float32)
    ob, sb, hc = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
    err = ctypes.create_string_buffer(512)
    st = R.gqref_gguf_load(os.fsencode(path), name.encode(), kind, _p(out), out.nbytes, ctypes.byref(ob), _p(sc),
                           sc.nbytes, ctypes.byref(sb), _p(hs), hs.nbytes, ctypes.byref(hc), err, 512)
    if st != 0:
        raise RuntimeError(f"reference load failed: {err.value.decode(errors='replace')}")
    return out[:ob.value].copy(), sc[:sb.value // 4].copy(), hs[:hc.value].copy()
