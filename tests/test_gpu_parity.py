"""GPU parity: libgq.so (HIP, gfx950) against the CPU oracle on the same seeded
inputs.  Dequantization and repack are bit-exact; GEMV/GEMM must be within
rel-L2 <= 1e-3 of the fp64-accumulated oracle."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3  # rel-L2 bound for GEMV / GEMM vs the fp64 oracle
FMTS = [O.Q4_0, O.Q8_0, O.Q4_K, O.Q4_K_GGML, O.Q6_K, O.Q6_K_GGML]


def bitexact(got, ref):
    """Bit-identical, except that any NaN equals any NaN (x86 and CDNA produce
    different default-NaN payloads for inf*0; the reference defines none)."""
    got = np.asarray(got, dtype=np.float32).ravel()
    ref = np.asarray(ref, dtype=np.float32).ravel()
    same = got.view(np.uint32) == ref.view(np.uint32)
    same |= np.isnan(got) & np.isnan(ref)
    return bool(same.all())


def _to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _bf16(a):
    """fp32 -> bf16 (round to nearest even) -> fp32."""
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def _special_scales(w, fmt):
    """Put fp16 edge values into the first blocks' scale fields."""
    w = w.copy()
    bb = O.BLOCK_BYTES[fmt]
    specials = [0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x7BFF, 0x7C00, 0xFC00, 0x7E00, 0x7C01, 0x8001, 0x3C00]
    nblk = w.size // bb
    for i, h in enumerate(specials[:nblk]):
        w[i * bb: i * bb + 2] = np.frombuffer(np.uint16(h).tobytes(), dtype=np.uint8)
        if fmt in (O.Q4_K, O.Q4_K_GGML):
            w[i * bb + 2: i * bb + 4] = np.frombuffer(np.uint16(specials[-1 - i]).tobytes(), dtype=np.uint8)
    return w


@pytest.mark.parametrize("fmt", FMTS)
def test_dequant_gguf_bitexact(dev, fmt):
    import gq
    n, k = 48, 1024
    w = _special_scales(O.gen_weights(fmt, n, k, seed=11 + fmt), fmt)
    ref = O.dequant(fmt, w)
    nb = w.size // O.BLOCK_BYTES[fmt]
    got = gq.dequant_gguf(fmt, _to_dev(w, dev), nb).cpu().numpy()
    assert bitexact(got, ref)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("shape", [(64, 1024), (40, 512), (7, 256), (1, 4096)])
def test_repack_device_matches_host_and_dequant(dev, fmt, shape):
    import gq
    n, k = shape
    w = _special_scales(O.gen_weights(fmt, n, k, seed=3 + n), fmt)
    host = gq.repack_host(fmt, w, n, k)
    d = gq.repack(fmt, _to_dev(w, dev), n, k).cpu().numpy()
    assert np.array_equal(host, d)
    back = gq.dequant_packed(fmt, _to_dev(host, dev), n, k).cpu().numpy().ravel()
    ref = O.dequant(fmt, w)
    assert bitexact(back, ref)


@pytest.mark.parametrize("fmt", FMTS)
def test_repack_rows_slices_in_any_order(dev, fmt):
    """Row slices repacked out of order into one buffer give the whole-tensor
    repack, including the zeroed padding rows of a ragged last tile."""
    import gq
    import torch
    n, k = 40, 1024
    w = O.gen_weights(fmt, n, k, seed=8 + fmt)
    rb = w.size // n
    out = torch.full((gq.packed_size(fmt, n, k),), 0xAB, dtype=torch.uint8, device=dev)
    for r0, rows in [(32, 8), (0, 16), (16, 16)]:
        gq.repack_rows(fmt, _to_dev(w[r0 * rb:(r0 + rows) * rb], dev), n, k, r0, rows, out)
    assert np.array_equal(out.cpu().numpy(), gq.repack_host(fmt, w, n, k))


def _gemv_case(dev, fmt, n, k, batch, seed):
    import gq
    w = O.gen_weights(fmt, n, k, seed=seed)
    x = O.gen_x(batch, k, seed=seed + 1)
    ref = O.gemv(fmt, w, x, n, k)
    packed = _to_dev(gq.repack_host(fmt, w, n, k), dev)
    y = gq.gemv(fmt, packed, _to_dev(x, dev), n, k).cpu().numpy()
    return O.rel_l2(y, ref)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("batch", [1, 2, 3, 4, 8, 9, 16])
def test_gemv_batches(dev, fmt, batch):
    err = _gemv_case(dev, fmt, 256, 2048, batch, seed=100 + batch)
    assert err <= TOL, err


@pytest.mark.parametrize("fmt", [O.Q4_0, O.Q8_0])
@pytest.mark.parametrize("shape", [(100, 288), (1, 32), (17, 96), (33, 160)])
def test_gemv_ragged_q32(dev, fmt, shape):
    n, k = shape
    err = _gemv_case(dev, fmt, n, k, 1, seed=7 + n)
    assert err <= TOL, err


@pytest.mark.parametrize("fmt", [O.Q4_K, O.Q4_K_GGML, O.Q6_K, O.Q6_K_GGML])
@pytest.mark.parametrize("shape", [(100, 256), (1, 768), (17, 512)])
def test_gemv_ragged_q4k(dev, fmt, shape):
    n, k = shape
    err = _gemv_case(dev, fmt, n, k, 2, seed=9 + n)
    assert err <= TOL, err


@pytest.mark.parametrize("fmt,n,k", [(O.Q4_0, 14336, 4096), (O.Q4_0, 4096, 14336), (O.Q8_0, 4096, 4096),
                                     (O.Q6_K, 32000, 4096),
                                     (O.Q4_K, 14336, 4096)])
def test_gemv_baseline_shapes(dev, fmt, n, k):
    err = _gemv_case(dev, fmt, n, k, 1, seed=1000 + fmt)
    assert err <= TOL, err


@pytest.mark.parametrize("fmt", [O.Q4_0, O.Q4_K])
@pytest.mark.parametrize("shape,batch", [((4096, 4096), 8), ((4096, 4096), 12), ((7168, 2048), 6),
                                         ((14336, 1024), 16), ((1000, 4096), 5), ((2048, 14336), 7)])
def test_gemv_batch_kernel_plans(dev, fmt, shape, batch):
    """Shapes that take each batch-kernel plan: one-stage with 8 and with 16
    staged rows, the windowed kernel, ragged rows, long K."""
    n, k = shape
    err = _gemv_case(dev, fmt, n, k, batch, seed=400 + batch)
    assert err <= TOL, err


@pytest.mark.parametrize("fmt,n,k,batch", [(O.Q4_K, 4096, 14336, 3), (O.Q4_K, 1000, 16384, 3),
                                           (O.Q4_0, 4096, 14336, 3), (O.Q8_0, 300, 14336, 3),
                                           (O.Q4_0, 700, 16384, 3), (O.Q4_0, 4096, 14336, 4),
                                           (O.Q4_K, 4096, 14336, 4)])
def test_gemv_long_k_small_batch(dev, fmt, n, k, batch):
    """Long K at batch 3..4: the int8 kernel stages its activation limbs for
    the batch rows present only and takes the shape where staging and static
    arrays fit the 160 KiB of a workgroup (batch 3 here); batch 4 at K =
    14336 does not fit and runs on the fp16 batch kernel."""
    err = _gemv_case(dev, fmt, n, k, batch, seed=500 + batch + fmt)
    assert err <= TOL, err


@pytest.mark.parametrize("fmt", [O.Q4_0, O.Q8_0, O.Q4_K, O.Q6_K])
@pytest.mark.parametrize("batch", [1, 3])
def test_gemv_long_k_falls_back(dev, fmt, batch):
    """K beyond the int8 kernel's registers (> 16384) runs on the fp16 kernel."""
    err = _gemv_case(dev, fmt, 48, 20480, batch, seed=300 + batch)
    assert err <= TOL, err


def test_gemv_special_inputs(dev):
    """All-8 nibbles -> zero weights; one-hot x selects a column."""
    import gq
    import torch
    n, k = 64, 512
    w = O.gen_weights(O.Q4_0, n, k, seed=5).reshape(-1, 18).copy()
    w[:, 2:] = 0x88
    packed = _to_dev(gq.repack_host(O.Q4_0, w.ravel(), n, k), dev)
    x = torch.randn(1, k, device=dev)
    # (q - 8) = 0 everywhere; the kernel applies the -8 offset as a separate
    # fp32 term, so allow its rounding (|d * x| ~ 1e-2 per term)
    assert torch.max(torch.abs(gq.gemv(O.Q4_0, packed, x, n, k))).item() <= 1e-5
    w2 = O.gen_weights(O.Q8_0, n, k, seed=6)
    p2 = _to_dev(gq.repack_host(O.Q8_0, w2, n, k), dev)
    W = O.dequant(O.Q8_0, w2).reshape(n, k)
    for col in (0, 37, k - 1):
        x = torch.zeros(1, k, device=dev)
        x[0, col] = 1.0
        y = gq.gemv(O.Q8_0, p2, x, n, k).cpu().numpy()[0]
        np.testing.assert_allclose(y, W[:, col], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("fmt", [O.Q4_0, O.Q8_0, O.Q4_K])
@pytest.mark.parametrize("m,n,k", [(64, 256, 1024), (130, 200, 512), (512, 512, 4096)])
def test_gemm_parity(dev, fmt, m, n, k):
    import gq
    import torch
    w = O.gen_weights(fmt, n, k, seed=50 + m)
    a = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16)
    ref = O.gemv(fmt, w, a.float().numpy(), n, k)
    packed = _to_dev(gq.repack_host(fmt, w, n, k), dev)
    c = gq.gemm(fmt, packed, a.to(dev), n, k).cpu().numpy()
    assert O.rel_l2(c, ref) <= TOL
    cb = gq.gemm(fmt, packed, a.to(dev), n, k, out_dtype=torch.bfloat16).float().cpu().numpy()
    assert np.array_equal(cb, _bf16(c))  # the fp32 result, rounded to nearest even


def test_gemm_f32_activations_and_matmul_routing(dev):
    import gq
    import torch
    fmt, n, k = O.Q4_0, 96, 512
    w = O.gen_weights(fmt, n, k, seed=77)
    packed = _to_dev(gq.repack_host(fmt, w, n, k), dev)
    for m in (1, 5, 16, 17, 33, 48, 49):
        a = O.gen_x(m, k, seed=m)
        ref = O.gemv(fmt, w, a, n, k)
        c = gq.matmul(fmt, packed, _to_dev(a, dev), n, k).cpu().numpy()
        assert O.rel_l2(c, ref) <= TOL, m


@pytest.mark.parametrize("fmt", [O.Q4_0, O.Q8_0, O.Q4_K])
@pytest.mark.parametrize("m", [17, 20, 36, 48])
def test_gemm_small_m_f32(dev, fmt, m):
    """gq_gemm with 16 < M <= 48, f32 A and C (the skinny kernel, one partial
    64-row block)."""
    import gq
    import torch
    n, k = 200, 1024
    w = O.gen_weights(fmt, n, k, seed=80 + m)
    a = O.gen_x(m, k, seed=90 + m)
    ref = O.gemv(fmt, w, a, n, k)
    packed = _to_dev(gq.repack_host(fmt, w, n, k), dev)
    c = gq.gemm(fmt, packed, _to_dev(a, dev), n, k, out_dtype=torch.float32).cpu().numpy()
    assert O.rel_l2(c, ref) <= TOL


@pytest.mark.parametrize("m,n,k", [(96, 160, 1024), (1, 16, 32), (130, 300, 4192), (257, 48, 224), (128, 256, 4096)])
def test_q8_i8_path(dev, m, n, k):
    """Int8 route: partial M / N tiles, a single block, and K % 128 != 0 (a
    last chunk with padding blocks, whose activation scales are zero)."""
    import gq
    import torch
    w = O.gen_weights(O.Q8_0, n, k, seed=21)
    a = O.gen_x(m, k, seed=22)
    qa, da = gq.quantize_act_q8(_to_dev(a, dev))
    rq, rd = O.quantize_act_q8(a)
    assert np.array_equal(qa.cpu().numpy(), rq)
    assert np.array_equal(da.cpu().numpy().view(np.uint32), rd.view(np.uint32))
    packed = _to_dev(gq.repack_host(O.Q8_0, w, n, k), dev)
    c = gq.gemm_q8_i8(packed, qa, da, n).cpu().numpy()
    ref = O.gemm_q8_i8(w, rq, rd, n)
    assert O.rel_l2(c, ref) <= 1e-5
    # error of activation quantization itself, vs the fp32-activation oracle
    assert O.rel_l2(c, O.gemv(O.Q8_0, w, a, n, k)) <= 2e-2


@pytest.mark.parametrize("m", [1, 4, 40])
def test_compat_int8_int4_launchers(dev, m):
    """Reference INT8 / INT4 launchers: the fp32 GEMV up to 32 rows (rel-L2
    1e-5); above, the reference's MFMA route on fp16 operands (weights * scale
    and A rounded to fp16, as gemm_kernels.hip:820-908 does: rel-L2 1e-3),
    unless force_gemv."""
    import gq
    n, k = 64, 256
    tol = 1e-5 if m <= 32 else TOL
    rng = np.random.default_rng(m)
    wf = rng.standard_normal((n, k)).astype(np.float32) * 0.05
    x = O.gen_x(m, k, seed=m + 1)
    q8, s8 = O.requant_int8(wf)
    ref8 = O.gemm_int8_wt(x, q8, s8, m, n, k)
    y8 = gq.launch_int8_wt(_to_dev(x, dev), _to_dev(q8, dev), _to_dev(s8, dev), m, n, k).cpu().numpy()
    assert O.rel_l2(y8, ref8) <= tol
    p4, s4 = O.requant_int4(wf)
    hs = O.head_scales(wf, 4, 16, k)
    ref4 = O.gemm_int4_wt(x, p4, s4, hs, m, n, k, 32, 16)
    y4 = gq.launch_int4_wt(_to_dev(x, dev), _to_dev(p4, dev), _to_dev(s4, dev), _to_dev(hs, dev), m, n, k,
                           head_dim=16).cpu().numpy()
    assert O.rel_l2(y4, ref4) <= tol
    y4g = gq.launch_int4_wt(_to_dev(x, dev), _to_dev(p4, dev), _to_dev(s4, dev), _to_dev(hs, dev), m, n, k,
                            head_dim=16, force_gemv=True).cpu().numpy()
    ref4g = O.gemm_int4_wt(x, p4, s4, hs, m, n, k, 32, 16, gemv_route=True)
    assert O.rel_l2(y4g, ref4g) <= 1e-5


@pytest.mark.parametrize("m,gs,fp16", [(100, 32, False), (33, 64, True), (300, 32, True), (64, 16, False)])
def test_compat_mfma_route(dev, m, gs, fp16):
    """M > 32: INT8 / INT4 weights converted to Q8_0 / Q4_0 blocks (head scales
    folded into d), repacked and run through gq_gemm; a group size that is not
    a multiple of 32 keeps the fp32 GEMV."""
    import gq
    n, k = 96, 512
    rng = np.random.default_rng(m + gs)
    x = O.gen_x(m, k, seed=m)
    q8 = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    s = (rng.random(n * k // gs + 2).astype(np.float32) + 0.5) * 0.01  # (+2: the row-based index of ragged K)
    tol = TOL if gs % 32 == 0 else 1e-5
    y8 = gq.launch_int8_wt(_to_dev(x, dev), _to_dev(q8, dev), _to_dev(s, dev), m, n, k, group_size=gs)
    assert O.rel_l2(y8.cpu().numpy(), O.gemm_int8_wt(x, q8, s, m, n, k, gs)) <= tol
    p4 = rng.integers(0, 256, size=(n * k // 2,), dtype=np.uint8)
    hs = (rng.random(n // 16).astype(np.float32) + 0.5)
    xa = x.astype(np.float16) if fp16 else x
    ref4 = O.gemm_int4_wt(xa.astype(np.float32), p4, s, hs, m, n, k, gs, 16)
    y4 = gq.launch_int4_wt(_to_dev(xa, dev), _to_dev(p4, dev), _to_dev(s, dev), _to_dev(hs, dev), m, n, k,
                           group_size=gs, head_dim=16)
    assert O.rel_l2(y4.cpu().numpy(), ref4) <= tol


@pytest.mark.parametrize("m,n,k,gs,hd", [(1, 70, 1040, 32, 10), (3, 33, 4096, 64, 0), (9, 16, 48, 16, 8),
                                         (5, 40, 100, 20, 0), (2, 24, 1024, 32, 8), (2, 40, 8192, 32, 0),
                                         (1, 20, 14336, 32, 4), (6, 17, 16400, 16, 0), (1, 8200, 512, 32, 8),
                                         (3, 30, 120, 48, 0), (40, 70, 1040, 32, 10), (40, 48, 1056, 64, 0),
                                         (36, 20, 120, 48, 0)])
def test_compat_launchers_shapes(dev, m, n, k, gs, hd):
    """Reference launchers: ragged rows, K past one 1024-k segment up to the
    LDS-staged GEMV's 16384 (and beyond: the per-wave form), other group sizes
    (K or gs not a multiple of 16: the per-element fallback kernel), head
    scales, fp16 activations for INT4.  K % gs != 0 (1040 / 32, 120 / 48,
    1056 / 64) checks the reference's scale index of each route: s_row[k/gs]
    with s_row = scales + (n*K)/gs up to 32 rows, scales[(n*K + k)/gs] above
    (the fp32 GEMV computes that form when the MFMA route's conditions fail,
    1040 and 120; 1056 / 64 takes the MFMA route, fp16 operands)."""
    import gq
    import torch
    rng = np.random.default_rng(n + k)
    wf = rng.standard_normal((n, k)).astype(np.float32) * 0.05
    x = O.gen_x(m, k, seed=k)
    q8 = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    s = (rng.random(n * k // gs + 2).astype(np.float32) + 0.5) * 0.01  # (+2: the row-based index of ragged K)
    tol = TOL if (m > 32 and k % 32 == 0 and gs % 32 == 0) else 1e-5
    ref8 = O.gemm_int8_wt(x, q8, s, m, n, k, gs)
    y8 = gq.launch_int8_wt(_to_dev(x, dev), _to_dev(q8, dev), _to_dev(s, dev), m, n, k, group_size=gs)
    assert O.rel_l2(y8.cpu().numpy(), ref8) <= tol
    p4 = rng.integers(0, 256, size=(n * k // 2,), dtype=np.uint8)
    hs = (rng.random(max(1, n // hd) if hd else 1).astype(np.float32) + 0.5) if hd else None
    ref4 = O.gemm_int4_wt(x, p4, s, hs, m, n, k, gs, hd)
    y4 = gq.launch_int4_wt(_to_dev(x, dev), _to_dev(p4, dev), _to_dev(s, dev),
                           _to_dev(hs, dev) if hs is not None else None, m, n, k, group_size=gs, head_dim=hd)
    assert O.rel_l2(y4.cpu().numpy(), ref4) <= tol
    xh = x.astype(np.float16)
    ref4h = O.gemm_int4_wt(xh.astype(np.float32), p4, s, hs, m, n, k, gs, hd)
    y4h = gq.launch_int4_wt(_to_dev(xh, dev), _to_dev(p4, dev), _to_dev(s, dev),
                            _to_dev(hs, dev) if hs is not None else None, m, n, k, group_size=gs, head_dim=hd)
    assert O.rel_l2(y4h.cpu().numpy(), ref4h) <= tol
    if m > 32:  # force_gemv: the GEMV route's scale index at any M
        y4g = gq.launch_int4_wt(_to_dev(x, dev), _to_dev(p4, dev), _to_dev(s, dev),
                                _to_dev(hs, dev) if hs is not None else None, m, n, k, group_size=gs, head_dim=hd,
                                force_gemv=True)
        ref4g = O.gemm_int4_wt(x, p4, s, hs, m, n, k, gs, hd, gemv_route=True)
        assert O.rel_l2(y4g.cpu().numpy(), ref4g) <= 1e-5


@pytest.mark.parametrize("tile", [12, 14])
def test_gemm_epilogue_very_wide_n(dev, tile, monkeypatch):
    """N so wide that a tile's C offsets (N x tile rows x 4 bytes) pass 2 GiB:
    the register-B kernel's epilogue takes its 64-bit address path instead of
    the buffer resource; f32 and bf16 C."""
    import gq
    import torch
    monkeypatch.setenv("GQ_GEMM_TILE", str(tile))
    fmt, m, n, k = O.Q4_0, 5, (1 << 21) + 48, 64
    w = O.gen_weights(fmt, n, k, seed=77)
    a = torch.randn(m, k, generator=torch.Generator().manual_seed(77)).to(torch.bfloat16)
    ref = O.gemv(fmt, w, a.float().numpy(), n, k)
    packed = _to_dev(gq.repack_host(fmt, w, n, k), dev)
    c = gq.gemm(fmt, packed, a.to(dev), n, k).cpu().numpy()
    assert O.rel_l2(c, ref) <= TOL
    cb = gq.gemm(fmt, packed, a.to(dev), n, k, out_dtype=torch.bfloat16).float().cpu().numpy()
    assert np.array_equal(cb, _bf16(c))


@pytest.mark.parametrize("tile,pd", [(0, 2), (0, 4), (1, 2), (2, 2), (3, 2), (4, 2), (4, 3), (4, 4), (5, 4),
                                     (6, 2), (6, 3), (6, 4), (7, 4), (8, 4), (9, 3), (9, 4), (10, 4), (11, 2),
                                     (11, 4), (12, 2), (12, 3), (13, 2), (13, 3), (13, 4), (14, 2), (14, 3), (14, 4),
                                     (15, 2), (15, 3), (15, 4), (16, 2), (16, 3), (17, 2), (17, 3), (17, 4),
                                     (18, 2), (18, 4)])
@pytest.mark.parametrize("fmt", [O.Q4_0, O.Q8_0, O.Q4_K])
def test_gemm_every_kernel_shape(dev, fmt, tile, pd, monkeypatch):
    """Each GEMM kernel / tile shape (forced through GQ_GEMM_TILE) and, for the
    register-B kernel, pipeline depths (GQ_GEMM_PD), on a shape with partial
    tiles in M and N.  15-18 split K among 2 or 4 wave groups of one
    workgroup (the groups' sums added through LDS); a depth whose LDS does not
    fit falls back to the deepest that does."""
    import gq
    import torch
    monkeypatch.setenv("GQ_GEMM_TILE", str(tile))
    monkeypatch.setenv("GQ_GEMM_PD", str(pd))
    m, n, k = 300, 400, 1024
    w = O.gen_weights(fmt, n, k, seed=60 + tile)
    a = torch.randn(m, k, generator=torch.Generator().manual_seed(tile)).to(torch.bfloat16)
    ref = O.gemv(fmt, w, a.float().numpy(), n, k)
    packed = _to_dev(gq.repack_host(fmt, w, n, k), dev)
    c = gq.gemm(fmt, packed, a.to(dev), n, k).cpu().numpy()
    assert O.rel_l2(c, ref) <= TOL


@pytest.mark.parametrize("fmt,k", [(O.Q4_0, 128), (O.Q8_0, 384), (O.Q4_K, 256), (O.Q4_K, 768), (O.Q4_0, 1536)])
@pytest.mark.parametrize("pd", [2, 3, 4])
def test_gemm_short_k_loops(dev, fmt, k, pd, monkeypatch):
    """K step counts of 2..24 (fewer steps than the pipeline is deep, and the
    unrolled step loops' guarded tails) for each pipeline depth; the K-group
    shapes also with one step per group, and with a step count the groups do
    not divide (the plan then takes the same tile without K groups)."""
    import gq
    import torch
    monkeypatch.setenv("GQ_GEMM_PD", str(pd))
    for tile in (4, 6, 11, 12, 13, 14, 15, 16, 17, 18):
        monkeypatch.setenv("GQ_GEMM_TILE", str(tile))
        m, n = 200, 160
        w = O.gen_weights(fmt, n, k, seed=70 + k)
        a = torch.randn(m, k, generator=torch.Generator().manual_seed(k)).to(torch.bfloat16)
        ref = O.gemv(fmt, w, a.float().numpy(), n, k)
        packed = _to_dev(gq.repack_host(fmt, w, n, k), dev)
        c = gq.gemm(fmt, packed, a.to(dev), n, k).cpu().numpy()
        assert O.rel_l2(c, ref) <= TOL, (tile, pd)


@pytest.mark.parametrize("fmt", [O.Q4_0, O.Q8_0, O.Q4_K, O.Q4_K_GGML])
@pytest.mark.parametrize("m,n,k", [(49, 200, 1024), (64, 4096, 4096), (100, 520, 2048), (256, 96, 512),
                                   (130, 1000, 256), (40, 300, 14336), (70, 48, 8192)])
def test_gemm_skinny(dev, fmt, m, n, k):
    """Few rows: the skinny GEMM (K split over a workgroup's 8 waves, or 16 on
    32-row blocks for long K; A in the fragments' order), partial row blocks
    and ragged row tiles, with bf16 and f32 activations and f32 / bf16 output
    (Q8_0 with long K takes the tiled kernel)."""
    import gq
    import torch
    w = O.gen_weights(fmt, n, k, seed=110 + m)
    a = torch.randn(m, k, generator=torch.Generator().manual_seed(m + n))
    packed = _to_dev(gq.repack_host(fmt, w, n, k), dev)
    for adt in (torch.bfloat16, torch.float32):
        aa = a.to(adt)
        ref = O.gemv(fmt, w, aa.float().numpy(), n, k)
        c = gq.gemm(fmt, packed, aa.to(dev), n, k).cpu().numpy()
        assert O.rel_l2(c, ref) <= TOL, adt
        cb = gq.gemm(fmt, packed, aa.to(dev), n, k, out_dtype=torch.bfloat16).float().cpu().numpy()
        assert np.array_equal(cb, _bf16(c)), adt


@pytest.mark.parametrize("k", [512, 4608])
def test_q6k_matmul(dev, k):
    """Q6_K, M > 16: gq_matmul runs the skinny GEMM (K <= 4096) or 16-row GEMV
    batches (longer K)."""
    import gq
    n, m = 96, 40
    w = O.gen_weights(O.Q6_K, n, k, seed=31)
    a = O.gen_x(m, k, seed=32)
    packed = _to_dev(gq.repack_host(O.Q6_K, w, n, k), dev)
    c = gq.matmul(O.Q6_K, packed, _to_dev(a, dev), n, k).cpu().numpy()
    assert O.rel_l2(c, O.gemv(O.Q6_K, w, a, n, k)) <= TOL


@pytest.mark.parametrize("fmt", [O.Q4_0, O.Q8_0])
@pytest.mark.parametrize("m,n,k", [(50, 33, 96), (33, 17, 288), (1, 16, 32), (7, 40, 160)])
def test_gemm_skinny_ragged_k(dev, fmt, m, n, k):
    """Skinny GEMM with K not a multiple of the 128-element chunk (zero-padded
    activations past K), fewer chunks than waves, and M below one row tile."""
    import gq
    import torch
    w = O.gen_weights(fmt, n, k, seed=120 + k)
    a = torch.randn(m, k, generator=torch.Generator().manual_seed(k)).to(torch.bfloat16)
    ref = O.gemv(fmt, w, a.float().numpy(), n, k)
    packed = _to_dev(gq.repack_host(fmt, w, n, k), dev)
    c = gq.gemm(fmt, packed, a.to(dev), n, k).cpu().numpy()
    assert O.rel_l2(c, ref) <= TOL


@pytest.mark.parametrize("fmt", [O.Q6_K, O.Q6_K_GGML])
@pytest.mark.parametrize("m,n", [(17, 300), (100, 2048), (300, 160)])
def test_gemm_q6k_skinny(dev, fmt, m, n):
    """gq_gemm on Q6_K (skinny kernel at any M, K <= 4096), bf16 A, f32 and
    bf16 C; longer K is refused."""
    import gq
    import torch
    k = 1024
    w = O.gen_weights(fmt, n, k, seed=33 + m)
    a = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16)
    ref = O.gemv(fmt, w, a.float().numpy(), n, k)
    packed = _to_dev(gq.repack_host(fmt, w, n, k), dev)
    c = gq.gemm(fmt, packed, a.to(dev), n, k).cpu().numpy()
    assert O.rel_l2(c, ref) <= TOL
    cb = gq.gemm(fmt, packed, a.to(dev), n, k, out_dtype=torch.bfloat16).float().cpu().numpy()
    assert np.array_equal(cb, _bf16(c))
    k2 = 4608
    w2 = O.gen_weights(fmt, 32, k2, seed=34)
    p2 = _to_dev(gq.repack_host(fmt, w2, 32, k2), dev)
    with pytest.raises(gq.GQError):
        gq.gemm(fmt, p2, torch.zeros(20, k2, dtype=torch.bfloat16, device=dev), 32, k2)


def test_binding_loads_before_torch(dev):
    """gq imported and loaded before torch in a fresh process still reaches the
    device (libgq and torch must share one HIP runtime)."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = ("import sys; sys.path[:0] = [%r, %r]\n"
            "import gq, numpy as np\n"
            "gq.load()\n"
            "import torch\n"
            "w = np.zeros(gq.gguf_bytes(gq.FMT_Q8_0, 16, 32), np.uint8)\n"
            "p = torch.from_numpy(gq.repack_host(gq.FMT_Q8_0, w, 16, 32)).cuda()\n"
            "y = gq.gemv(gq.FMT_Q8_0, p, torch.ones(1, 32, device='cuda'), 16, 32)\n"
            "assert float(y.abs().sum()) == 0.0\n"
            "print('ok')\n") % (os.path.join(root, "gretacore-v3_amd"), os.path.join(root, "oracle"))
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0 and "ok" in out.stdout, out.stderr[-2000:]
