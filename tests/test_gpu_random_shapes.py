"""Seeded random shapes through every public GEMV / GEMM entry point against
the fp64 oracle: ragged N (any row count, partial 16-row tiles), K at every
block granularity the format allows (short, long, not a multiple of the
kernels' 128 / 256-element chunks), batch 1..16, M from the batch-GEMV band
to several tiles, bf16 / fp16 / fp32 activations, rows scaled by 1e-3..1e3,
and the fused entry points (batch 1..4) with and without RMSNorm.  The
shapes come from a fixed seed, so each case id names one reproducible
problem, and the plan the library picked is printed with the case.

Bound: rel-L2 <= 1e-3 over the whole output once each
batch row is divided by the scale it was given, and row by row for rows of at
least 64 outputs.  A row of a few outputs is a sample too small for rel-L2:
the fp16 batch kernels' rounding (weights and activations each to 11
significant bits, ~5e-4 rel-L2 on long rows) can reach 1.2e-3 on a row of 4
(Q6_K, N = 4, K = 6400, batch 14), so such rows are held to 3e-3 each."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _k(rng, fmt, kmax):
    be = O.BLOCK_ELEMS[fmt]
    return be * int(rng.integers(1, kmax // be + 1))


def _row_scales(rng, rows):
    return (10.0 ** rng.uniform(-3, 3, size=(rows, 1))).astype(np.float32)


def _check(y, ref, scales):
    """y, ref [rows][n]; scales [rows][1]: the bound of the module docstring."""
    y = np.asarray(y, dtype=np.float64) / scales
    ref = np.asarray(ref, dtype=np.float64) / scales
    assert O.rel_l2(y, ref) <= TOL
    row_tol = TOL if y.shape[1] >= 64 else 3 * TOL
    for b in range(y.shape[0]):
        assert O.rel_l2(y[b], ref[b]) <= row_tol, b


def _gemv_cases():
    rng = np.random.default_rng(20261202)
    fmts = [O.Q4_0, O.Q8_0, O.Q4_K, O.Q4_K_GGML, O.Q6_K, O.Q6_K_GGML]
    out = []
    for i in range(48):
        fmt = fmts[i % len(fmts)]
        k = _k(rng, fmt, 9216)
        n = int(rng.integers(1, max(2, min(3000, 6_000_000 // k))))
        out.append((i, fmt, n, k, int(rng.integers(1, 17))))
    return out


def _gemm_cases():
    rng = np.random.default_rng(20261203)
    fmts = [O.Q4_0, O.Q8_0, O.Q4_K, O.Q4_K_GGML]
    out = []
    for i in range(32):
        fmt = fmts[i % len(fmts)]
        k = _k(rng, fmt, 6144)
        n = int(rng.integers(1, max(2, min(2000, 4_000_000 // k))))
        m = int(rng.integers(17, 700))
        out.append((i, fmt, m, n, k, int(rng.integers(0, 3))))
    return out


def _fused_cases():
    rng = np.random.default_rng(20261204)
    fmts = [O.Q4_0, O.Q8_0, O.Q4_K]
    out = []
    for i in range(18):
        fmt = fmts[i % len(fmts)]
        k = _k(rng, fmt, 8192)
        ns = [int(rng.integers(1, 1500)) for _ in range(int(rng.integers(1, 5)))]
        out.append((i, fmt, ns, k, int(rng.integers(1, 5)), bool(i % 2)))
    return out


@pytest.mark.parametrize("case", _gemv_cases(), ids=lambda c: f"gemv{c[0]}")
def test_random_gemv(dev, case):
    import gq
    i, fmt, n, k, batch = case
    rng = np.random.default_rng(1000 + i)
    print(f"random gemv {i}: fmt={fmt} n={n} k={k} batch={batch} plan={gq.gemv_plan(fmt, n, k, batch)}",
          flush=True)
    w = O.gen_weights(fmt, n, k, seed=2000 + i)
    sc = _row_scales(rng, batch)
    x = O.gen_x(batch, k, seed=3000 + i) * sc
    y = gq.gemv(fmt, gq.repack(fmt, _dev(w, dev), n, k), _dev(x, dev), n, k).cpu().numpy()
    _check(y, O.gemv(fmt, w, x, n, k), sc)


@pytest.mark.parametrize("case", _gemm_cases(), ids=lambda c: f"gemm{c[0]}")
def test_random_gemm(dev, case):
    import torch

    import gq
    i, fmt, m, n, k, adt = case
    rng = np.random.default_rng(4000 + i)
    dt = [torch.bfloat16, torch.float16, torch.float32][adt]
    print(f"random gemm {i}: fmt={fmt} m={m} n={n} k={k} a={dt}", flush=True)
    w = O.gen_weights(fmt, n, k, seed=5000 + i)
    sc = _row_scales(rng, m)
    a = torch.from_numpy(O.gen_x(m, k, seed=6000 + i) * sc).to(dt)
    packed = gq.repack(fmt, _dev(w, dev), n, k)
    c = gq.gemm(fmt, packed, a.to(dev), n, k).cpu().numpy()
    _check(c, O.gemv(fmt, w, a.float().numpy(), n, k), sc)
    if i % 4 == 0:  # bf16 C: the fp32 result rounded once
        cb = gq.gemm(fmt, packed, a.to(dev), n, k, out_dtype=torch.bfloat16).float().cpu().numpy()
        assert np.array_equal(cb, torch.from_numpy(c).to(torch.bfloat16).float().numpy())


@pytest.mark.parametrize("case", _fused_cases(), ids=lambda c: f"fused{c[0]}")
def test_random_fused(dev, case):
    import gq
    i, fmt, ns, k, batch, norm = case
    rng = np.random.default_rng(7000 + i)
    print(f"random fused {i}: fmt={fmt} ns={ns} k={k} batch={batch} norm={norm}", flush=True)
    ws = [O.gen_weights(fmt, n, k, seed=8000 + 10 * i + j) for j, n in enumerate(ns)]
    sc = _row_scales(rng, batch)
    x = O.gen_x(batch, k, seed=9000 + i) * sc
    gamma = (0.5 + rng.random(k)).astype(np.float32) if norm else None
    eps = 1e-5
    xr = O.rmsnorm(x, gamma, eps).astype(np.float32) if norm else x
    mats = [(gq.repack(fmt, _dev(w, dev), n, k), n) for w, n in zip(ws, ns)]
    ys = gq.gemv_multi(fmt, mats, _dev(x, dev), k, gamma=_dev(gamma, dev) if norm else None, eps=eps)
    # (after RMSNorm every row has unit scale)
    osc = np.ones_like(sc) if norm else sc
    for w, n, y in zip(ws, ns, ys):
        _check(y.cpu().numpy(), O.gemv(fmt, w, xr, n, k), osc)
    # SwiGLU: gate = the first matrix, up = another of the same N
    n = ns[0]
    wg, wu = ws[0], O.gen_weights(fmt, n, k, seed=8500 + i)
    y = gq.gemv_swiglu(fmt, mats[0][0], gq.repack(fmt, _dev(wu, dev), n, k), _dev(x, dev), n, k,
                       gamma=_dev(gamma, dev) if norm else None, eps=eps).cpu().numpy()
    ref = O.swiglu(O.gemv(fmt, wg, xr, n, k), O.gemv(fmt, wu, xr, n, k))
    # silu(g) u is not linear in x: its rows are compared as they are
    _check(y, ref, np.ones_like(sc))
