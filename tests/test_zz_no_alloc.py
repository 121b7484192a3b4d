"""gq_gemm_static (the allocation-free gq_gemm) against gq_gemm, called
through the C ABI: two calls in a row on one GPU, the second with a smaller
input, each bit-identical to gq_gemm with a caller workspace (the same
kernels on the same data); a shape whose conversion exceeds the fixed scratch
is refused, and the same size with no conversion to make is accepted."""
import ctypes

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def _run_static(lib, fmt, packed, a, n, k, out_dtype):
    import torch

    import gq
    m = a.shape[0]
    c = torch.full((m, n), float("nan"), dtype=out_dtype, device=a.device)
    dt = {torch.bfloat16: gq.DT_BF16, torch.float16: gq.DT_F16, torch.float32: gq.DT_F32}[a.dtype]
    cdt = gq.DT_F32 if out_dtype == torch.float32 else gq.DT_BF16
    st = lib.gq_gemm_static(fmt, ctypes.c_void_p(packed.data_ptr()), ctypes.c_void_p(a.data_ptr()), dt,
                            ctypes.c_void_p(c.data_ptr()), cdt, m, n, k,
                            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    return st, c


def test_gemm_static_matches_gemm(dev):
    import torch

    import gq
    lib = gq.load()
    assert lib.gq_gemm_static_max_bytes() == 64 << 20
    cases = [(O.Q4_0, 1024, 4096, 4096, torch.bfloat16, torch.float32),   # tiled kernel
             (O.Q4_K, 200, 1024, 2048, torch.float32, torch.bfloat16),   # smaller: tiled, other format
             (O.Q8_0, 48, 512, 1024, torch.bfloat16, torch.float32)]     # smaller again: skinny kernel
    for i, (fmt, m, n, k, adt, odt) in enumerate(cases):
        w = O.gen_weights(fmt, n, k, seed=500 + i)
        packed = gq.repack(fmt, torch.from_numpy(w).to(dev), n, k)
        a = torch.randn(m, k, generator=torch.Generator().manual_seed(600 + i)).to(adt).to(dev)
        ref = gq.gemm(fmt, packed, a, n, k, out_dtype=odt, workspace=gq.Workspace(dev, 0))
        st, c = _run_static(lib, fmt, packed, a, n, k, odt)
        assert st == 0, gq.load().gq_status_string(st)
        torch.cuda.synchronize()
        assert torch.equal(c, ref), i
        if odt == torch.float32:
            assert O.rel_l2(c.cpu().numpy(), O.gemv(fmt, w, a.float().cpu().numpy(), n, k)) <= 1e-3
    # beyond the scratch: refused, nothing launched
    m, k = 8192, 4096
    assert gq.gemm_workspace_bytes(O.Q4_0, m, k) > lib.gq_gemm_static_max_bytes()
    a = torch.zeros(m, k, dtype=torch.bfloat16, device=dev)
    packed = torch.zeros(gq.packed_size(O.Q4_0, 16, k), dtype=torch.uint8, device=dev)
    st, _ = _run_static(lib, O.Q4_0, packed, a, 16, k, torch.float32)
    assert st == 4  # GQ_ERR_WORKSPACE
    # the same size needs no scratch when A is used as it is (fp16 of the
    # padded width, Q8_0's k order): accepted, bit-identical to gq_gemm
    n = 512
    w = O.gen_weights(O.Q8_0, n, k, seed=510)
    packed = gq.repack(O.Q8_0, torch.from_numpy(w).to(dev), n, k)
    a = torch.randn(m, k, generator=torch.Generator().manual_seed(610)).to(torch.float16).to(dev)
    assert gq.gemm_workspace_bytes(O.Q8_0, m, k) > lib.gq_gemm_static_max_bytes()
    ref = gq.gemm(O.Q8_0, packed, a, n, k, out_dtype=torch.float32)
    st, c = _run_static(lib, O.Q8_0, packed, a, n, k, torch.float32)
    assert st == 0, gq.load().gq_status_string(st)
    torch.cuda.synchronize()
    assert torch.equal(c, ref)
