"""GPU parity of the fused decode GEMVs (gq_gemv_multi, gq_gemv_swiglu): the
quantized counterparts of the reference's fused RMSNorm+QKV and FFN-front
kernels (fused_compute_kernels.hip:22-243), against the fp64 oracle
(rmsnorm, gemv, swiglu) within rel-L2 1e-3."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _packed(fmt, n, k, seed, dev):
    import gq
    w = O.gen_weights(fmt, n, k, seed)
    return w, gq.repack(fmt, _dev(w, dev), n, k)


@pytest.mark.parametrize("fmt", [O.Q4_0, O.Q8_0, O.Q4_K])
@pytest.mark.parametrize("batch", [1, 2, 3, 4])
@pytest.mark.parametrize("norm", [False, True])
def test_gemv_multi_qkv(dev, fmt, batch, norm):
    import gq
    k = 1024
    ns = [512, 128, 128]  # q, k, v with 4x fewer kv rows (GQA)
    mats, ws = [], []
    for i, n in enumerate(ns):
        w, p = _packed(fmt, n, k, 40 + i, dev)
        ws.append(w)
        mats.append((p, n))
    x = O.gen_x(batch, k, 7)
    gamma = (np.random.default_rng(8).standard_normal(k) * 0.5 + 1.0).astype(np.float32)
    eps = 1e-5
    ys = gq.gemv_multi(fmt, mats, _dev(x, dev), k, gamma=_dev(gamma, dev) if norm else None, eps=eps)
    xin = O.rmsnorm(x, gamma, eps).astype(np.float32) if norm else x
    for w, (p, n), y in zip(ws, mats, ys):
        ref = O.gemv(fmt, w, xin, n, k)
        assert O.rel_l2(y.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("fmt", [O.Q4_0, O.Q4_K])
def test_gemv_multi_matches_single_calls_shapes(dev, fmt):
    """Four matrices of ragged row counts, long K."""
    import gq
    k = 2048
    ns = [48, 16, 300, 1000]
    mats, ws = [], []
    for i, n in enumerate(ns):
        w, p = _packed(fmt, n, k, 60 + i, dev)
        ws.append(w)
        mats.append((p, n))
    x = O.gen_x(2, k, 9)
    ys = gq.gemv_multi(fmt, mats, _dev(x, dev), k)
    for w, (p, n), y in zip(ws, mats, ys):
        assert O.rel_l2(y.cpu().numpy(), O.gemv(fmt, w, x, n, k)) <= TOL


@pytest.mark.parametrize("fmt", [O.Q4_0, O.Q8_0, O.Q4_K])
@pytest.mark.parametrize("batch", [1, 4])
@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("n", [512, 200])
def test_gemv_swiglu(dev, fmt, batch, norm, n):
    import gq
    k = 1024
    wg, pg = _packed(fmt, n, k, 70, dev)
    wu, pu = _packed(fmt, n, k, 71, dev)
    x = O.gen_x(batch, k, 11)
    gamma = (np.random.default_rng(12).standard_normal(k) * 0.5 + 1.0).astype(np.float32)
    y = gq.gemv_swiglu(fmt, pg, pu, _dev(x, dev), n, k, gamma=_dev(gamma, dev) if norm else None, eps=1e-6)
    xin = O.rmsnorm(x, gamma, 1e-6).astype(np.float32) if norm else x
    g = O.gemv(fmt, wg, xin, n, k).astype(np.float64)
    u = O.gemv(fmt, wu, xin, n, k).astype(np.float64)
    ref = O.swiglu(g, u)
    assert O.rel_l2(y.cpu().numpy(), ref) <= TOL


def test_fused_reject_bad_args(dev):
    import gq
    _, p = _packed(O.Q4_0, 64, 256, 1, dev)
    x = _dev(O.gen_x(5, 256, 1), dev)
    with pytest.raises(gq.GQError):
        gq.gemv_multi(O.Q4_0, [(p, 64)], x, 256)  # batch 5 is not supported by the fused path
    with pytest.raises(gq.GQError):
        gq.gemv_swiglu(O.Q4_0, p, p, x, 64, 256)


@pytest.mark.parametrize("fmt", [O.Q4_0, O.Q8_0, O.Q4_K])
@pytest.mark.parametrize("norm", [False, True])
def test_fused_fallback_long_k(dev, fmt, norm):
    """Shapes one fused launch cannot stage: batch 4 with K = 16384 (gq_gemv_multi
    and gq_gemv_swiglu) and K = 14336 at batch 1 for gq_gemv_swiglu (its
    gate/up chunk lists exceed a wave's registers).  The plans report the
    fallback (zeros) and the calls give the fused forms' results: RMSNorm,
    one GEMV per matrix, silu(gate) * up."""
    import gq
    eps = 1e-5
    for k, batch, multi in ((16384, 4, True), (16384, 4, False), (14336, 1, False)):
        print(f"fused fallback fmt={fmt} k={k} batch={batch} multi={multi} norm={norm}", flush=True)
        x = O.gen_x(batch, k, 21) * 3.0
        gamma = (np.random.default_rng(22).standard_normal(k) * 0.5 + 1.0).astype(np.float32)
        xin = O.rmsnorm(x, gamma, eps).astype(np.float32) if norm else x
        g = _dev(gamma, dev) if norm else None
        if multi:
            ns = [300, 64, 1000]
            assert gq.gemv_multi_plan(fmt, ns, k, batch) == (0, 0, 0)
            pw = [_packed(fmt, n, k, 80 + i, dev) for i, n in enumerate(ns)]
            ys = gq.gemv_multi(fmt, [(p, n) for (_, p), n in zip(pw, ns)], _dev(x, dev), k, gamma=g, eps=eps)
            for (w, _), n, y in zip(pw, ns, ys):
                assert O.rel_l2(y.cpu().numpy(), O.gemv(fmt, w, xin, n, k)) <= TOL
        else:
            n = 200
            assert gq.gemv_swiglu_plan(fmt, n, k, batch) == (0, 0)
            wg, pg = _packed(fmt, n, k, 90, dev)
            wu, pu = _packed(fmt, n, k, 91, dev)
            y = gq.gemv_swiglu(fmt, pg, pu, _dev(x, dev), n, k, gamma=g, eps=eps).cpu().numpy()
            ref = O.swiglu(O.gemv(fmt, wg, xin, n, k), O.gemv(fmt, wu, xin, n, k))
            assert O.rel_l2(y, ref) <= TOL


@pytest.mark.parametrize("fmt", [O.Q6_K, O.Q6_K_GGML])
@pytest.mark.parametrize("batch", [1, 3])
def test_fused_q6k(dev, fmt, batch):
    """Q6_K (Q4_K_M files keep some projections in it): the fused entry points
    take the fallback (plans report zeros) and match the oracle, with RMSNorm."""
    import gq
    k, eps = 1024, 1e-5
    ns = [256, 64]
    pw = [_packed(fmt, n, k, 95 + i, dev) for i, n in enumerate(ns)]
    x = O.gen_x(batch, k, 23)
    gamma = (np.random.default_rng(24).standard_normal(k) * 0.5 + 1.0).astype(np.float32)
    xin = O.rmsnorm(x, gamma, eps).astype(np.float32)
    assert gq.gemv_multi_plan(fmt, ns, k, batch) == (0, 0, 0)
    ys = gq.gemv_multi(fmt, [(p, n) for (_, p), n in zip(pw, ns)], _dev(x, dev), k, gamma=_dev(gamma, dev), eps=eps)
    for (w, _), n, y in zip(pw, ns, ys):
        assert O.rel_l2(y.cpu().numpy(), O.gemv(fmt, w, xin, n, k)) <= TOL
    assert gq.gemv_swiglu_plan(fmt, ns[0], k, batch) == (0, 0)
    wu, pu = _packed(fmt, ns[0], k, 99, dev)
    y = gq.gemv_swiglu(fmt, pw[0][1], pu, _dev(x, dev), ns[0], k, gamma=_dev(gamma, dev), eps=eps).cpu().numpy()
    ref = O.swiglu(O.gemv(fmt, pw[0][0], xin, ns[0], k), O.gemv(fmt, wu, xin, ns[0], k))
    assert O.rel_l2(y, ref) <= TOL
