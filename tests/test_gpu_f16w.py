"""FP16-weight route (the reference's GretaCompute::gemm with FP16 B,
greta_compute_hip.cpp:361-371 -> launch_gemm_mixed_f16f32 /
launch_gemm_mfma_mixed_f16f32, gemm_kernels.hip:294-358, 387-523):
C = A W^T with fp32 A, fp16 W [N][K] row-major, fp32 C.  Checked against an
fp64 numpy product of the same fp16 weights (rel-L2 <= 1e-3 per row, the
north-star bound), at batch 1..16, ragged N and K, more than 16 rows of A,
activations beyond fp16's range, the lm_head shape, and through the two
reference launchers (the same kernels: bit-identical to gq_gemm_f16w)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _w(n, k, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((n, k)) * 0.05).astype(np.float16)


def _ref(w16, a):
    return np.asarray(a, dtype=np.float64) @ w16.astype(np.float64).T


def _rel(y, ref):
    return float(np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-300))


def _run(dev, w16, a):
    import torch

    import gq
    w = torch.from_numpy(w16).to(dev)
    x = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)
    return gq.gemm_f16w(w, x, w16.shape[0], w16.shape[1]).cpu().numpy()


@pytest.mark.parametrize("n,k,m", [(4096, 4096, 1), (4096, 4096, 4), (4096, 4096, 8), (4096, 4096, 16),
                                   (14336, 4096, 1), (1000, 4096, 3), (4096, 4160, 5), (512, 14336, 2),
                                   (1024, 2048, 17), (768, 4096, 40), (4096, 1024, 16)])
def test_f16w_matches_fp64(dev, n, k, m):
    w16 = _w(n, k, seed=n + k + m)
    a = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)
    y = _run(dev, w16, a)
    ref = _ref(w16, a)
    assert np.isfinite(y).all()
    for r in range(m):
        assert _rel(y[r], ref[r]) <= TOL, r


@pytest.mark.parametrize("m", [1, 5, 16])
def test_f16w_wide_range_activations(dev, m):
    """Spikes of 1e5 (beyond fp16's 65504) in every 32-block and a row of
    ~1e-6: finite outputs, every row within 1e-3 of the fp64 product."""
    n, k = 2048, 4096
    w16 = _w(n, k, seed=77)
    rng = np.random.default_rng(100 + m)
    a = rng.standard_normal((m, k)).astype(np.float32)
    pos = rng.integers(0, 32, size=(m, k // 32)) + 32 * np.arange(k // 32)[None, :]
    for r in range(m):
        a[r, pos[r]] = (rng.choice([-1.0, 1.0], size=k // 32) * 1e5).astype(np.float32)
    if m > 1:
        a[m - 1] = (rng.standard_normal(k) * 1e-6).astype(np.float32)
    y = _run(dev, w16, a)
    ref = _ref(w16, a)
    assert np.isfinite(y).all()
    for r in range(m):
        assert _rel(y[r], ref[r]) <= TOL, r


def test_f16w_lm_head_shape(dev):
    """The reference's decode lm_head on FP16 weights (a Q6_K output.weight
    dequantized to fp16, weight_loader.cpp:573-666): 128256 x 4096, batch 1;
    checked on 4096 sampled rows of W."""
    import torch

    import gq
    n, k = 128256, 4096
    g = torch.Generator(device="cpu").manual_seed(5)
    w = (torch.randn(n, k, generator=g) * 0.05).to(torch.float16)
    a = np.random.default_rng(6).standard_normal((1, k)).astype(np.float32)
    y = gq.gemm_f16w(w.to(dev), torch.from_numpy(a).to(dev), n, k).cpu().numpy()
    rows = np.linspace(0, n - 1, 4096).astype(int)
    ref = _ref(w[rows].numpy(), a)
    assert _rel(y[:, rows], ref) <= TOL


def test_reference_f16_launchers(dev):
    """launch_gemm_mixed_f16f32 / launch_gemm_mfma_mixed_f16f32 under their
    argument lists: the same results as gq_gemm_f16w; K == 0 writes zeros on
    the VALU launcher and leaves C alone on the MFMA one (the reference's
    early return); strides other than lda = K, ldc = N are refused."""
    import torch

    import gq
    n, k = 1024, 2048
    w16 = _w(n, k, seed=3)
    w = torch.from_numpy(w16).to(dev)
    for m in (5, 48):
        a = torch.from_numpy(np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)).to(dev)
        ref = gq.gemm_f16w(w, a, n, k)
        for mfma in (False, True):
            c = gq.launch_mixed_f16f32(a, w, m, n, k, mfma=mfma)
            assert torch.equal(c, ref), (m, mfma)
    a = torch.zeros((4, 32), device=dev)
    c = torch.full((4, n), 7.0, device=dev)
    gq.launch_mixed_f16f32(a, w, 4, n, 0, mfma=True, c=c)
    torch.cuda.synchronize()
    assert bool((c == 7.0).all())
    gq.launch_mixed_f16f32(a, w, 4, n, 0, mfma=False, c=c)
    torch.cuda.synchronize()
    assert bool((c == 0.0).all())
    lib = gq.load()
    st = lib.gq_launch_gemm_mixed_f16f32(gq._stream(None), gq._ptr(a), gq._ptr(w), gq._ptr(c), 4, n, 32, 64, n, n)
    assert st == 2  # GQ_ERR_UNSUPPORTED


@pytest.mark.parametrize("n,k,m", [(300, 40, 3), (1000, 100, 17), (77, 8, 1), (513, 4104, 5)])
def test_f16w_any_k_and_alignment(dev, n, k, m):
    """K not a multiple of 32 (the reference's FP16 launchers take any K) and
    operands not 16-byte aligned run the plain fp32-accumulating kernel:
    rel-L2 <= 1e-5 against the fp64 product of the same fp16 weights (fp32
    activations, fp32 sums), through gq_gemm_f16w and both reference launchers."""
    import torch

    import gq
    w16 = _w(n, k, seed=n + k)
    a = np.random.default_rng(k).standard_normal((m, k)).astype(np.float32)
    ref = _ref(w16, a)
    y = _run(dev, w16, a)
    assert _rel(y, ref) <= 1e-5
    for mfma in (False, True):
        c = gq.launch_mixed_f16f32(torch.from_numpy(a).to(dev), torch.from_numpy(w16).to(dev), m, n, k, mfma=mfma)
        assert _rel(c.cpu().numpy(), ref) <= 1e-5
    # K % 32 == 0 but the operands start 4 bytes into their buffers
    k2 = 64
    w2 = _w(n, k2, seed=7)
    a2 = np.random.default_rng(8).standard_normal((m, k2)).astype(np.float32)
    wb = torch.zeros(n * k2 + 8, dtype=torch.float16, device=dev)
    ab = torch.zeros(m * k2 + 4, dtype=torch.float32, device=dev)
    wv, av = wb[2:2 + n * k2].view(n, k2), ab[1:1 + m * k2].view(m, k2)
    wv.copy_(torch.from_numpy(w2))
    av.copy_(torch.from_numpy(a2))
    c2 = gq.gemm_f16w(wv, av, n, k2).cpu().numpy()
    assert _rel(c2, _ref(w2, a2)) <= 1e-5
