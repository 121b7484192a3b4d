"""CPU tests of the C ABI: libgq.so loads, exports every function declared in
include/*.h, validates its arguments, and the host-side repack is lossless.
No compute call here needs a GPU."""
import ctypes
import glob
import os
import re
import subprocess

import numpy as np
import pytest

import gq
import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for m in re.finditer(r"\b(gq[a-z0-9_]*)\s*\(", text):
            names.add(m.group(1))
    return names


def exported_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", gq.LIB_PATH], capture_output=True, text=True, check=True)
    return {line.split()[-1] for line in out.stdout.splitlines() if " T " in line}


def test_library_exports_every_declared_symbol():
    gq.load()
    decl = declared_functions()
    assert len(decl) >= 20
    missing = decl - exported_symbols()
    assert not missing, f"declared but not exported: {sorted(missing)}"
    lib = ctypes.CDLL(gq.LIB_PATH)
    for name in decl:
        assert getattr(lib, name) is not None


def test_python_binding_covers_the_c_abi():
    missing = declared_functions() - set(gq.exported_symbols())
    assert not missing, f"declared in include/*.h but not bound in gq.py: {sorted(missing)}"


def test_status_strings_and_version():
    lib = gq.load()
    assert lib.gq_abi_version() == 1
    for s in range(6):
        assert lib.gq_status_string(s)
    assert lib.gq_status_string(99) == b"unknown status"


ALL = [gq.FMT_Q4_0, gq.FMT_Q8_0, gq.FMT_Q4_K, gq.FMT_Q4_K_GGML, gq.FMT_Q6_K, gq.FMT_Q6_K_GGML]


@pytest.mark.parametrize("fmt", ALL)
def test_sizes_match_gguf(fmt):
    # bytes per weight are unchanged by the repack when the shape is tile-aligned
    for n, k in [(4096, 4096), (14336, 4096), (4096, 14336), (1024, 4096)]:
        assert gq.packed_size(fmt, n, k) == gq.gguf_bytes(fmt, n, k)
    assert gq.gguf_bytes(gq.FMT_Q4_0, 14336, 4096) == 33030144
    assert gq.gguf_bytes(gq.FMT_Q8_0, 128256, 4096) == 558170112
    assert gq.gguf_bytes(gq.FMT_Q6_K, 128256, 4096) == 128256 * 16 * 210


@pytest.mark.parametrize("fmt", ALL)
@pytest.mark.parametrize("shape", [(64, 1024), (7, 256), (40, 512), (1, 4096), (17, 2304)])
def test_host_repack_roundtrip(fmt, shape):
    n, k = shape
    if k % O.BLOCK_ELEMS[fmt]:
        pytest.skip("K not a multiple of the block")
    w = O.gen_weights(fmt, n, k, seed=n + k)
    p = gq.repack_host(fmt, w, n, k)
    assert p.size >= w.size
    assert np.array_equal(gq.unpack_host(fmt, p, n, k), w)


def test_repack_is_a_permutation_of_the_bits():
    # every GGUF byte (and every nibble) lands somewhere: popcount is preserved
    n, k = 32, 1024
    for fmt in (gq.FMT_Q4_0, gq.FMT_Q8_0, gq.FMT_Q4_K, gq.FMT_Q6_K, gq.FMT_Q6_K_GGML):
        w = O.gen_weights(fmt, n, k, seed=1)
        p = gq.repack_host(fmt, w, n, k)
        assert np.unpackbits(p).sum() == np.unpackbits(w).sum()


def test_argument_validation():
    lib = gq.load()
    buf = (ctypes.c_uint8 * 64)()
    out = ctypes.c_size_t(0)
    assert lib.gq_packed_size(99, 16, 32, ctypes.byref(out)) == 2          # unknown format
    assert lib.gq_packed_size(gq.FMT_Q4_0, 16, 33, ctypes.byref(out)) == 1  # K not a block multiple
    assert lib.gq_packed_size(gq.FMT_Q4_K, 16, 128, ctypes.byref(out)) == 1
    assert lib.gq_packed_size(gq.FMT_Q4_0, 1 << 25, 32, ctypes.byref(out)) == 1
    assert lib.gq_repack_host(gq.FMT_Q4_0, None, 16, 32, buf) == 1
    assert lib.gq_gemv(gq.FMT_Q4_0, buf, buf, buf, 16, 32, 0, None, 0, None) == 2    # batch 0
    assert lib.gq_gemv(gq.FMT_Q4_0, buf, buf, buf, 16, 32, 17, None, 0, None) == 2   # batch 17
    assert lib.gq_gemv(gq.FMT_Q4_0, None, buf, buf, 16, 32, 1, None, 0, None) == 1
    assert lib.gq_gemm(gq.FMT_Q4_0, buf, buf, 7, buf, 0, 4, 16, 32, None, 0, None) == 2  # bad dtype
    assert lib.gq_gemv_workspace_bytes(gq.FMT_Q4_0, 4096, 17) == 0
    assert lib.gq_gemv_workspace_bytes(gq.FMT_Q4_0, 4096, 4) > 0
    # Q6_K: GEMV (fp16 kernel, no workspace), GEMM for K <= 4096 only, no split
    # or fused GEMV
    assert lib.gq_gemv_workspace_bytes(gq.FMT_Q6_K, 4096, 4) == 0
    assert lib.gq_gemm(gq.FMT_Q6_K, buf, buf, 2, buf, 0, 32, 16, 4608, None, 0, None) == 2
    assert lib.gq_gemv_prep(gq.FMT_Q6_K, buf, 256, 1, buf, 64, None) == 2
    # row slices: whole tiles from a multiple of 16, or the tensor's end
    assert lib.gq_repack_rows(gq.FMT_Q4_0, buf, 40, 32, 8, 16, buf, None) == 1   # row0 not a tile start
    assert lib.gq_repack_rows(gq.FMT_Q4_0, buf, 40, 32, 0, 8, buf, None) == 1    # partial tile mid-tensor
    assert lib.gq_repack_rows(gq.FMT_Q4_0, buf, 40, 32, 32, 16, buf, None) == 1  # past the end
    assert lib.gq_repack_rows(gq.FMT_Q4_0, buf, 40, 32, 32, 0, buf, None) == 0   # empty slice: no-op
    # zero-sized problems are no-ops that need no device
    assert lib.gq_gemv(gq.FMT_Q4_0, buf, buf, buf, 0, 32, 1, None, 0, None) == 0
    assert lib.gq_gemm(gq.FMT_Q4_0, buf, buf, 2, buf, 0, 0, 16, 32, None, 0, None) == 0
    assert lib.gq_launch_gemm_mfma_int8_wt_fp32_acc32(None, buf, buf, buf, None, 0, 4, 4, 4, 4, 4, 32) == 0
    # int8 Q8_0 route: K a block multiple, activation rows 16-byte aligned
    base = ctypes.addressof(buf)
    qa16 = ctypes.c_void_p((base + 15) & ~15)
    qa_odd = ctypes.c_void_p(((base + 15) & ~15) + 1)
    assert lib.gq_gemm_q8_i8(buf, qa16, buf, buf, 4, 16, 33, None) == 1   # K not a block multiple
    assert lib.gq_gemm_q8_i8(buf, qa_odd, buf, buf, 4, 16, 32, None) == 1  # misaligned activations
    assert lib.gq_gemm_q8_i8(buf, None, buf, buf, 4, 16, 32, None) == 1
    assert lib.gq_gemm_q8_i8(buf, qa16, buf, buf, 0, 16, 32, None) == 0   # empty: no-op


def test_product_path_never_loads_the_oracle():
    """The shipped library must not link or reference the CPU oracle."""
    deps = subprocess.run(["ldd", gq.LIB_PATH], capture_output=True, text=True).stdout
    assert "gqoracle" not in deps and "gqref" not in deps
    src = open(os.path.join(ROOT, "gretacore-v3_amd", "gq.py")).read()
    assert "oracle" not in src.replace("no CPU fallback", "")


def test_calibration_library_is_separate():
    """The benchmark's calibration kernels (read probe, empty kernel) live in
    lib/libgqcalib.so, which exports them and needs nothing from libgq.so;
    the product library does not carry them."""
    calib = os.path.join(os.path.dirname(gq.LIB_PATH), "libgqcalib.so")
    defined = subprocess.run(["nm", "-D", "--defined-only", calib], capture_output=True, text=True,
                             check=True).stdout
    assert "gq_probe_read" in defined and "gq_probe_empty" in defined
    undef = subprocess.run(["nm", "-D", "-u", calib], capture_output=True, text=True, check=True).stdout
    assert "gq_" not in undef
    assert not any("probe" in s for s in exported_symbols())
