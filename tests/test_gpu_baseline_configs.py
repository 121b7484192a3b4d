"""GPU parity at the benchmark configurations' real sizes, and on activations
with outliers and a wide dynamic range.

Every shape the benchmark measures runs here against the fp64 oracle
(rel-L2 <= 1e-3).  bf16 outputs must equal the
kernel's own fp32 result rounded to nearest even, bit for bit, so the bf16
store adds exactly one rounding to a result that is itself within 1e-3 of
the oracle (a comparison with the oracle rounded to bf16 would instead count
the rounding-boundary flips that a 2e-4 difference in fp32 causes: ~8e-4 of
rel-L2 on its own).  Shapes:
  * Q8_0 GEMV 4096 x 4096, batch 1 (the CPU-path configuration);
  * Q4_0 decode GEMV 4096 x 4096, 14336 x 4096, 4096 x 14336, batch 1;
  * Q4_K 14336 x 4096 at batch 1, 4, 8, 16;
  * prefill GEMM M in {512, 2048} x (N x K) in {4096 x 4096, 14336 x 4096} for
    Q4_0, Q8_0 and Q4_K, bf16 A, f32 and bf16 C (rows sampled for the oracle);
  * the decode-step shapes: Q4_K 4096 x 14336, 1024 x 4096, 4096 x 4096, the
    Q8_0 lm_head 128256 x 4096, and the fused q/k/v (4096 / 1024 / 1024 x 4096)
    and gate/up (14336 x 4096) launches with and without the RMSNorm weight.
"""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _packed(fmt, w, n, k, dev):
    """Device repack (bit-exact with the host repack, tested elsewhere): the
    host repack of the largest tensors takes longer than the upload."""
    import gq
    return gq.repack(fmt, _dev(w, dev), n, k)


def _to_bf16(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def outlier_x(batch, k, seed, spike=300.0, tiny=1e-6, tiny_row=True):
    """N(0,1) rows with, in every 32-block, two entries of magnitude `spike`
    (random sign) and four entries of magnitude ~`tiny`; with tiny_row, one
    row of the batch (if batch > 1) is ~1e-5 throughout."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((batch, k)).astype(np.float32)
    nb = k // 32
    for b in range(batch):
        for j, cnt, mag in ((0, 2, spike), (1, 4, tiny)):
            pos = rng.integers(0, 32, size=(nb, cnt)) + 32 * np.arange(nb)[:, None]
            sgn = rng.choice([-1.0, 1.0], size=pos.shape)
            x[b, pos.ravel()] = (sgn * mag * (1.0 + rng.random(pos.shape))).ravel().astype(np.float32)
    if batch > 1 and tiny_row:
        x[batch - 1] = (rng.standard_normal(k) * 1e-5).astype(np.float32)
    return x


def _gemv_err(dev, fmt, n, k, batch, seed, x=None):
    import gq
    w = O.gen_weights(fmt, n, k, seed=seed)
    if x is None:
        x = O.gen_x(batch, k, seed=seed + 1000)
    y = gq.gemv(fmt, _packed(fmt, w, n, k, dev), _dev(x, dev), n, k).cpu().numpy()
    return O.rel_l2(y, O.gemv(fmt, w, x, n, k)), y, w, x


# ---- decode GEMV -------------------------------------------------------------
@pytest.mark.parametrize("fmt,n,k,batch", [
    (O.Q8_0, 4096, 4096, 1),
    (O.Q4_0, 4096, 4096, 1), (O.Q4_0, 14336, 4096, 1), (O.Q4_0, 4096, 14336, 1),
    (O.Q4_K, 14336, 4096, 1), (O.Q4_K, 14336, 4096, 4), (O.Q4_K, 14336, 4096, 8), (O.Q4_K, 14336, 4096, 16),
    (O.Q4_K, 4096, 14336, 1), (O.Q4_K, 1024, 4096, 1), (O.Q4_K, 4096, 4096, 1),
    (O.Q8_0, 128256, 4096, 1),
])
def test_gemv_benchmark_shapes(dev, fmt, n, k, batch):
    err = _gemv_err(dev, fmt, n, k, batch, seed=1000 + fmt + batch)[0]
    assert err <= TOL, err


@pytest.mark.parametrize("fmt,n,k,batch", [
    (O.Q4_0, 14336, 4096, 1), (O.Q8_0, 4096, 4096, 2), (O.Q4_K, 4096, 14336, 4),
    (O.Q4_K, 14336, 4096, 8), (O.Q4_0, 4096, 4096, 16),
])
def test_gemv_outlier_activations(dev, fmt, n, k, batch):
    """Per-32-block outliers (|x| 300-600) and near-zero entries: the int8
    two-limb split (batch <= 4) scales per 32-block, so its error follows the
    block's largest entry (there the last batch row is ~1e-5 throughout and
    is checked on its own)."""
    x = outlier_x(batch, k, seed=7 + batch, tiny_row=batch <= 2)
    err, y, w, _ = _gemv_err(dev, fmt, n, k, batch, seed=2000 + fmt, x=x)
    assert err <= TOL, err
    ref = O.gemv(fmt, w, x, n, k)
    for b in range(batch):
        assert O.rel_l2(y[b], ref[b]) <= TOL, b


@pytest.mark.parametrize("fmt", [O.Q4_0, O.Q8_0, O.Q4_K])
@pytest.mark.parametrize("n,k", [(14336, 4096), (4096, 14336), (1024, 4096)])
@pytest.mark.parametrize("batch", [3, 4, 5, 8, 16])
def test_gemv_wide_range_activations(dev, fmt, n, k, batch):
    """Activations beyond fp16's range and far below 1 through every batch
    GEMV kernel: spikes of 1e3..1e5 in every 32-block (beyond fp16's 65504),
    entries of ~1e-6, and one batch row of ~1e-6 throughout.  The fp16 batch
    kernels (batch 5..16; 3..4 where the int8 kernel's staging or registers do
    not fit) scale each batch row's 256-k window by a power of two before the
    fp16 rounding and restore it on the window's dot products, so outputs stay
    finite and every row -- the ~1e-6 row too -- is within 1e-3 of the fp64
    oracle, as the reference's fp32 GEMV band is (gemm_kernels.hip:594-634,
    763-817).  Shapes: 896 row tiles (the windowed kernel), 4096 x 14336 (long
    K), 1024 rows (the one-stage kernel)."""
    import gq
    spike = (1e3, 1e4, 1e5)[batch % 3]
    x = outlier_x(batch, k, seed=11 + batch + k, spike=spike)
    x[batch - 1] = (np.random.default_rng(batch).standard_normal(k) * 1e-6).astype(np.float32)
    w = O.gen_weights(fmt, n, k, seed=2100 + fmt)
    y = gq.gemv(fmt, _packed(fmt, w, n, k, dev), _dev(x, dev), n, k).cpu().numpy()
    assert np.isfinite(y).all()
    ref = O.gemv(fmt, w, x, n, k)
    for b in range(batch):
        assert O.rel_l2(y[b], ref[b]) <= TOL, b


@pytest.mark.parametrize("fmt", [O.Q4_0, O.Q8_0, O.Q4_K])
@pytest.mark.parametrize("batch", [1, 2])
def test_gemv_int8_limbs_spike_per_block(dev, fmt, batch):
    """The int8 two-limb GEMV (batch 1..2): N(0,1) rows with one 1e4 spike in
    every 32-block.  The limb step is the block's max / 32258, so the N(0,1)
    entries next to a spike carry an absolute error of up to ~0.3; each row
    must still be within 1e-3 of the fp64 oracle."""
    import gq
    n, k = 4096, 4096
    rng = np.random.default_rng(90 + batch)
    x = rng.standard_normal((batch, k)).astype(np.float32)
    pos = rng.integers(0, 32, size=(batch, k // 32)) + 32 * np.arange(k // 32)[None, :]
    for b in range(batch):
        x[b, pos[b]] = (rng.choice([-1.0, 1.0], size=k // 32) * 1e4).astype(np.float32)
    w = O.gen_weights(fmt, n, k, seed=2200 + fmt)
    y = gq.gemv(fmt, _packed(fmt, w, n, k, dev), _dev(x, dev), n, k).cpu().numpy()
    ref = O.gemv(fmt, w, x, n, k)
    for b in range(batch):
        assert O.rel_l2(y[b], ref[b]) <= TOL, b


# ---- prefill GEMM ------------------------------------------------------------
def _gemm_check(dev, fmt, m, n, k, a_bf16, seed, nrows=48):
    import torch

    import gq
    w = O.gen_weights(fmt, n, k, seed=seed)
    packed = _packed(fmt, w, n, k, dev)
    a = a_bf16.to(dev)
    rows = np.unique(np.linspace(0, m - 1, nrows).astype(int))
    a_rows = a_bf16[rows].float().numpy()
    ref = O.gemv(fmt, w, a_rows, n, k)
    c = gq.gemm(fmt, packed, a, n, k).cpu().numpy()
    err = O.rel_l2(c[rows], ref)
    cb = gq.gemm(fmt, packed, a, n, k, out_dtype=torch.bfloat16).float().cpu().numpy()
    return err, np.array_equal(cb, _to_bf16(c))


@pytest.mark.parametrize("fmt", [O.Q4_0, O.Q8_0, O.Q4_K])
@pytest.mark.parametrize("m,n,k", [(512, 4096, 4096), (512, 14336, 4096), (2048, 4096, 4096), (2048, 14336, 4096)])
def test_gemm_benchmark_shapes(dev, fmt, m, n, k):
    """The prefill configurations: 448 workgroups of 256 x 256 at 2048 x 14336
    (two rounds on 256 CUs, the XCD remap), 128 x 256 tiles at M = 512 and
    2048 x 4096, bf16 A ~ N(0,1), f32 C and bf16 C."""
    import torch
    a = torch.randn(m, k, generator=torch.Generator().manual_seed(2004 + m)).to(torch.bfloat16)
    err, bf16_exact = _gemm_check(dev, fmt, m, n, k, a, seed=1004 + fmt)
    assert err <= TOL, err
    assert bf16_exact


def wide_range_a(m, k, seed):
    """bf16 rows spanning many binades: N(0,1) rows with spikes of 1e3..1e5
    (beyond fp16's 65504), rows scaled to ~1e-6, and one row of 1e4-scale
    values throughout."""
    import torch
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(m, k, generator=g)
    spikes = torch.randint(0, k, (m, 8), generator=g)
    mags = 10.0 ** (3 + 2 * torch.rand(m, 8, generator=g))
    sgn = torch.where(torch.rand(m, 8, generator=g) < 0.5, -1.0, 1.0)
    a.scatter_(1, spikes, mags * sgn)
    a[1::7] *= 1e-6
    a[m // 2] = torch.randn(k, generator=g) * 1e4
    return a.to(torch.bfloat16)


@pytest.mark.parametrize("fmt", [O.Q4_0, O.Q8_0, O.Q4_K])
@pytest.mark.parametrize("m,n,k", [(2048, 4096, 4096), (64, 4096, 4096), (40, 512, 14336)])
def test_gemm_wide_range_activations(dev, fmt, m, n, k):
    """Activations beyond fp16's range (spikes to 1e5) and far below 1: the
    conversion to fp16 scales each row by a power of two (the product's
    exponent is restored on C), so neither overflows nor flushes; the tiled
    kernel (2048 rows), the skinny kernel (64 rows) and its 16-wave long-K form
    (40 x 14336) are covered.  Each sampled row is checked on its own too."""
    import torch

    import gq
    a = wide_range_a(m, k, seed=m + n)
    w = O.gen_weights(fmt, n, k, seed=3000 + fmt)
    packed = _packed(fmt, w, n, k, dev)
    rows = np.unique(np.concatenate([np.linspace(0, m - 1, 24).astype(int), [1, 8, m // 2]]))
    ref = O.gemv(fmt, w, a[rows].float().numpy(), n, k)
    call = gq.gemm(fmt, packed, a.to(dev), n, k).cpu().numpy()
    c = call[rows]
    assert np.isfinite(call).all()
    assert O.rel_l2(c, ref) <= TOL
    for i in range(len(rows)):
        assert O.rel_l2(c[i], ref[i]) <= TOL, rows[i]
    cb = gq.gemm(fmt, packed, a.to(dev), n, k, out_dtype=torch.bfloat16).float().cpu().numpy()
    assert np.array_equal(cb, _to_bf16(call))


# ---- fused decode launches at Llama-3-8B shapes ------------------------------
@pytest.mark.parametrize("fmt", [O.Q4_0, O.Q8_0, O.Q4_K])
@pytest.mark.parametrize("batch", [1, 4])
@pytest.mark.parametrize("norm", [False, True])
def test_fused_llama_shapes(dev, fmt, batch, norm):
    """gq_gemv_multi on q/k/v (4096 / 1024 / 1024 x 4096) and gq_gemv_swiglu on
    gate/up (14336 x 4096), K = 4096, with and without the RMSNorm weight:
    the launch plans (K split, row tiles) of the real decode shapes."""
    import gq
    k, eps = 4096, 1e-5
    rng = np.random.default_rng(batch + 10 * norm)
    x = O.gen_x(batch, k, seed=50 + batch) * 3.0
    gamma = (0.5 + rng.random(k)).astype(np.float32) if norm else None
    xn = O.rmsnorm(x, gamma, eps) if norm else x
    ns = (4096, 1024, 1024)
    ws = [O.gen_weights(fmt, n, k, seed=60 + i) for i, n in enumerate(ns)]
    ys = gq.gemv_multi(fmt, [(_packed(fmt, w, n, k, dev), n) for w, n in zip(ws, ns)], _dev(x, dev), k,
                       gamma=_dev(gamma, dev) if norm else None, eps=eps)
    for y, w, n in zip(ys, ws, ns):
        assert O.rel_l2(y.cpu().numpy(), O.gemv(fmt, w, xn, n, k)) <= TOL, n
    n = 14336
    wg = O.gen_weights(fmt, n, k, seed=70)
    wu = O.gen_weights(fmt, n, k, seed=71)
    y = gq.gemv_swiglu(fmt, _packed(fmt, wg, n, k, dev), _packed(fmt, wu, n, k, dev), _dev(x, dev), n, k,
                       gamma=_dev(gamma, dev) if norm else None, eps=eps).cpu().numpy()
    ref = O.swiglu(O.gemv(fmt, wg, xn, n, k), O.gemv(fmt, wu, xn, n, k))
    assert O.rel_l2(y, ref) <= TOL


@pytest.mark.parametrize("m,n,k", [(512, 4096, 4096), (2048, 14336, 4096)])
def test_gemm_q8_i8_benchmark_shapes(dev, m, n, k):
    """The int8 route of the prefill configuration (Q8_0, activations quantized
    per 32-block) at its real size: quantization bit-exact against the
    oracle's rule on every row, the GEMM against the exact integer block sums
    (fp64 scale products) on sampled rows, each row on its own too."""
    import torch

    import gq
    a = torch.randn(m, k, generator=torch.Generator().manual_seed(7000 + m)).to(torch.bfloat16)
    w = O.gen_weights(O.Q8_0, n, k, seed=7100 + m)
    packed = _packed(O.Q8_0, w, n, k, dev)
    qa, da = gq.quantize_act_q8(a.to(dev))
    rq, rd = O.quantize_act_q8(a.float().numpy())
    assert np.array_equal(qa.cpu().numpy(), rq)
    assert np.array_equal(da.cpu().numpy().view(np.uint32), rd.view(np.uint32))
    c = gq.gemm_q8_i8(packed, qa, da, n).cpu().numpy()
    assert np.isfinite(c).all()
    rows = np.unique(np.concatenate([np.linspace(0, m - 1, 12).astype(int), [127, 128, m - 1]]))
    ref = O.gemm_q8_i8(w, rq[rows], rd[rows], n)
    assert O.rel_l2(c[rows], ref) <= 1e-5
    for i in range(len(rows)):
        assert O.rel_l2(c[rows[i]], ref[i]) <= 1e-5, rows[i]
