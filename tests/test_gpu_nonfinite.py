"""Non-finite activations.  The reference's GEMV/GEMM accumulate in fp32
(gemv_kernels.hip, gemm_kernels.hip), so a NaN in a batch row makes every
output of that row NaN, and an Inf makes every output of the row non-finite
(+-Inf, NaN where the weight is zero or Infs of both signs meet).  Here the
row that holds the bad value must come out non-finite in exactly the
positions the fp64 oracle's do -- NaN where it gives NaN for a NaN input --
and every other batch row must stay finite and within the parity bound.
Covered: the int8 two-limb GEMV (batch 1-4), the fp16 batch GEMV (batch 8),
the GEMM (batch 64) and the decode chain.  The int8 path gives NaN, not
+-Inf, for an Inf input: its block scale is then Inf and the limbs zero."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-3
N, K = 256, 4096


def _dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("fmt", [O.Q4_0, O.Q8_0, O.Q4_K])
@pytest.mark.parametrize("batch", [1, 2, 4, 8, 64])
@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
def test_nonfinite_activation(dev, fmt, batch, bad):
    import gq
    print(f"nonfinite fmt={fmt} batch={batch} bad={bad}", flush=True)
    w = O.gen_weights(fmt, N, K, seed=1)
    p = gq.repack(fmt, _dev(w, dev), N, K)
    x = O.gen_x(batch, K, seed=2)
    x[0, 100] = bad
    xd = _dev(x, dev)
    y = (gq.gemv(fmt, p, xd, N, K) if batch <= 8 else gq.gemm(fmt, p, xd, N, K)).cpu().numpy()
    ref = O.gemv(fmt, w, x, N, K)
    assert np.array_equal(np.isfinite(y[0]), np.isfinite(ref[0]))
    if np.isnan(bad):
        assert np.isnan(y[0]).all()
    if batch > 1:
        assert np.isfinite(y[1:]).all()
        assert O.rel_l2(y[1:], ref[1:]) <= TOL


@pytest.mark.parametrize("bad", [np.nan, np.inf])
def test_nonfinite_chain(dev, bad):
    import torch

    import gq
    print(f"nonfinite chain bad={bad}", flush=True)
    fmt = O.Q4_K
    w = O.gen_weights(fmt, N, K, seed=3)
    p = gq.repack(fmt, _dev(w, dev), N, K)
    x = O.gen_x(1, K, seed=4)
    x[0, 3000] = bad
    y = torch.zeros(N, device=dev)
    ch = gq.Chain(fmt, [{"w": p, "x": _dev(x[0], dev), "y": y, "N": N, "K": K}], dev)
    ch.run()
    torch.cuda.synchronize()
    assert ch.error() == 0
    assert np.isnan(y.cpu().numpy()).all()
