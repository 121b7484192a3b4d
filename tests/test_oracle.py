"""CPU tests that pin the oracle (oracle/gq_oracle.c) before it is trusted as
the checker of the HIP path: golden vectors produced by the reference's own
functions, hand-built known-answer blocks, closed forms and brute force."""
import os

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def bits_equal(a, b):
    a = np.asarray(a, np.float32).ravel()
    b = np.asarray(b, np.float32).ravel()
    same = a.view(np.uint32) == b.view(np.uint32)
    return bool((same | (np.isnan(a) & np.isnan(b))).all())


# ---- fp16 -----------------------------------------------------------------------
def test_fp16_to_fp32_exhaustive_vs_reference_golden():
    ref = np.load(os.path.join(GOLD, "fp16_ref.npz"))["out"]
    L = O.lib()
    got = np.array([L.gqo_fp16_to_fp32(h) for h in range(65536)], dtype=np.float32)
    assert bits_equal(got, ref)


def test_fp16_to_fp32_matches_ieee_except_nan():
    L = O.lib()
    h = np.arange(65536, dtype=np.uint16)
    got = np.array([L.gqo_fp16_to_fp32(int(i)) for i in h], dtype=np.float32)
    ieee = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ieee)
    assert bits_equal(got[~nan], ieee[~nan])
    # reference quirk (weight_loader.cpp:105): exponent 31 -> +-Inf, payload dropped
    assert np.all(np.isinf(got[nan]))
    assert np.all(np.signbit(got[nan]) == ((h[nan] >> 15) == 1))


def test_float_to_half_rne_matches_numpy_for_normals():
    L = O.lib()
    rng = np.random.default_rng(0)
    v = (rng.standard_normal(20000) * np.exp(rng.uniform(-9, 10, 20000))).astype(np.float32)
    v = v[(np.abs(v) > 6.2e-5) & (np.abs(v) < 65000)]
    got = np.array([L.gqo_float_to_half(float(x)) for x in v], dtype=np.uint16)
    assert np.array_equal(got, v.astype(np.float16).view(np.uint16))


@pytest.mark.skipif(not O.ref_available(), reason="reference harness not built")
def test_float_to_half_matches_reference_cpu_reference():
    L, R = O.lib(), O.ref()
    rng = np.random.default_rng(1)
    v = (rng.standard_normal(5000) * np.exp(rng.uniform(-20, 12, 5000))).astype(np.float32)
    for x in v:
        assert L.gqo_float_to_half(float(x)) == R.gqref_float_to_half(float(x))


# ---- Q4_K (reference layout) -------------------------------------------------
def test_q4k_reference_golden():
    g = np.load(os.path.join(GOLD, "q4k_ref.npz"))
    assert bits_equal(O.dequant(O.Q4_K, g["blocks"]), g["out"])


@pytest.mark.skipif(not O.ref_available(), reason="reference harness not built")
def test_q4k_against_reference_function_random():
    R = O.ref()
    w = O.gen_weights(O.Q4_K, 64, 4096, seed=5)
    ref = np.empty(64 * 4096, np.float32)
    R.gqref_dequant_q4_k(w.ctypes.data, w.size // 144, ref.ctypes.data)
    assert bits_equal(O.dequant(O.Q4_K, w), ref)


def _q4k_block(d, dmin, sc, m, q, ggml=False):
    """Hand-assemble a Q4_K block from codes (the inverse of the unpacking
    written out independently of the oracle)."""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.float16(dmin).tobytes(), np.uint8)
    s = np.zeros(12, np.uint8)
    if not ggml:
        for j in range(4):
            s[j] = sc[j] | ((sc[4 + j] & 3) << 6)
            s[6 + j] = m[j] | ((m[4 + j] & 3) << 6)
        s[4] = (sc[4] >> 2) | ((sc[5] >> 2) << 4)
        s[5] = (sc[6] >> 2) | ((sc[7] >> 2) << 4)
        s[10] = (m[4] >> 2) | ((m[5] >> 2) << 4)
        s[11] = (m[6] >> 2) | ((m[7] >> 2) << 4)
        for j in range(8):
            for l in range(16):
                b[16 + 16 * j + l] = q[32 * j + 2 * l] | (q[32 * j + 2 * l + 1] << 4)
    else:
        for j in range(4):
            s[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
            s[j + 4] = m[j] | ((m[j + 4] >> 4) << 6)
            s[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
        for p in range(4):
            for l in range(32):
                b[16 + 32 * p + l] = q[64 * p + l] | (q[64 * p + 32 + l] << 4)
    b[4:16] = s
    return b


@pytest.mark.parametrize("ggml", [False, True])
def test_q4k_hand_built_block(ggml):
    rng = np.random.default_rng(7 + ggml)
    sc = rng.integers(0, 64, 8)
    m = rng.integers(0, 64, 8)
    q = rng.integers(0, 16, 256)
    d, dmin = 0.5, 0.25  # exact in fp16: every product and difference is exact
    blk = _q4k_block(d, dmin, sc, m, q, ggml)
    got = O.dequant(O.Q4_K_GGML if ggml else O.Q4_K, blk)
    want = np.array([d * sc[i // 32] * q[i] - dmin * m[i // 32] for i in range(256)], np.float32)
    assert np.array_equal(got, want)


def test_q4k_layouts_differ():
    """The reference layout is not llama.cpp's: the same bytes decode differently."""
    w = O.gen_weights(O.Q4_K, 4, 256, seed=3)
    assert not np.array_equal(O.dequant(O.Q4_K, w), O.dequant(O.Q4_K_GGML, w))


def test_q4k_codes_cover_0_63():
    # d = 1, dmin = 0, every nibble 1: the output is the scale code itself
    rng = np.random.default_rng(2)
    blocks = []
    for _ in range(64):
        sc = rng.integers(0, 64, 8)
        blocks.append(_q4k_block(1.0, 0.0, sc, np.zeros(8, int), np.ones(256, int)))
    out = O.dequant(O.Q4_K, np.concatenate(blocks)).reshape(64, 8, 32)
    codes = out[:, :, 0]
    assert codes.min() >= 0 and codes.max() <= 63 and len(np.unique(codes)) > 40
    assert np.all(out == out[:, :, :1])


# ---- Q6_K (next-tier, reference layout) -----------------------------------------
def test_q6k_reference_golden():
    g = np.load(os.path.join(GOLD, "q6k_ref.npz"))
    assert bits_equal(O.dequant(O.Q6_K, g["blocks"]), g["out"])


def _q6k_block(d, sc, codes, ggml):
    """Pack 256 six-bit codes into a Q6_K block (the inverse of the two
    layouts' decoders, written element by element)."""
    b = np.zeros(210, np.uint8)
    for i, c in enumerate(codes):
        lo, hi = int(c) & 15, int(c) >> 4
        if not ggml:
            b[i // 2] |= lo << (4 * (i % 2))
            b[128 + i // 4] |= hi << (2 * (i % 4))
        else:
            h, k, l = i // 128, (i // 32) % 4, i % 32
            b[64 * h + l + 32 * (k % 2)] |= lo << (4 * (k // 2))
            b[128 + 32 * h + l] |= hi << (2 * k)
    b[192:208] = np.asarray(sc, np.int8).view(np.uint8)
    b[208:210] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    return b


@pytest.mark.parametrize("ggml", [False, True])
def test_q6k_hand_built_block(ggml):
    rng = np.random.default_rng(11 + ggml)
    codes = rng.integers(0, 64, 256)
    sc = rng.integers(-128, 128, 16)
    d = 0.25  # exact: every product is exact in fp32
    got = O.dequant(O.Q6_K_GGML if ggml else O.Q6_K, _q6k_block(d, sc, codes, ggml))
    want = np.array([(d * (codes[i] - 32)) * sc[i // 16] for i in range(256)], np.float32)
    assert np.array_equal(got, want)


def test_q6k_layouts_differ():
    w = O.gen_weights(O.Q6_K, 4, 256, seed=3)
    assert not np.array_equal(O.dequant(O.Q6_K, w), O.dequant(O.Q6_K_GGML, w))


def test_q6k_extremes():
    # codes 0 and 63 -> -32 d sc and 31 d sc; sc = -128 .. 127
    codes = np.array([0, 63] * 128)
    sc = np.array([-128, 127] * 8)
    for ggml in (False, True):
        y = O.dequant(O.Q6_K_GGML if ggml else O.Q6_K, _q6k_block(1.0, sc, codes, ggml))
        assert y[0] == 4096.0 and y[1] == -3968.0 and y[16] == -4064.0 and y[17] == 3937.0


# ---- Q4_0 / Q8_0 (GGUF spec) ------------------------------------------------------
def test_q4_0_known_answer():
    # byte j = j | (15 - j) << 4, d = 0.5: y[j] = (j - 8)/2, y[j + 16] = (7 - j)/2
    b = np.zeros(18, np.uint8)
    b[0:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    for j in range(16):
        b[2 + j] = j | ((15 - j) << 4)
    y = O.dequant(O.Q4_0, b)
    want = [(j - 8) / 2 for j in range(16)] + [(7 - j) / 2 for j in range(16)]
    assert np.array_equal(y, np.array(want, np.float32))


def test_q4_0_all_eight_is_zero_and_d_scales():
    w = O.gen_weights(O.Q4_0, 8, 256, seed=1).reshape(-1, 18).copy()
    w[:, 2:] = 0x88
    assert np.all(O.dequant(O.Q4_0, w) == 0)
    w2 = O.gen_weights(O.Q4_0, 8, 256, seed=1).reshape(-1, 18).copy()
    d = w2[:, 0:2].copy().view(np.float16).astype(np.float32)
    w2[:, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    ints = O.dequant(O.Q4_0, w2).reshape(-1, 32)
    assert np.all(ints == np.round(ints)) and ints.min() >= -8 and ints.max() <= 7
    w3 = O.gen_weights(O.Q4_0, 8, 256, seed=1)
    assert np.array_equal(O.dequant(O.Q4_0, w3).reshape(-1, 32), (ints * d).astype(np.float32))


def test_q8_0_known_answer():
    b = np.zeros(34, np.uint8)
    b[0:2] = np.frombuffer(np.float16(-0.25).tobytes(), np.uint8)
    q = np.array([-127, -1, 0, 1, 127] + list(range(-13, 14)), np.int8)
    b[2:] = q.view(np.uint8)
    assert np.array_equal(O.dequant(O.Q8_0, b), (q.astype(np.float32) * -0.25))


# ---- matmul oracle ----------------------------------------------------------------
def test_gemm_ref_known_answer_from_reference_test():
    # tools/bench/runtime/src/cpu_ref_test.cpp:8-24
    C = O.gemm_ref(np.array([[1, 2], [3, 4]], np.float32), np.array([[5, 6], [7, 8]], np.float32))
    assert C.tolist() == [[19, 22], [43, 50]]


def test_gemm_ref_golden():
    g = np.load(os.path.join(GOLD, "gemm_ref.npz"))
    assert np.array_equal(O.gemm_ref(g["A"], g["B"]), g["C"])


@pytest.mark.parametrize("fmt", [O.Q4_0, O.Q8_0, O.Q4_K, O.Q4_K_GGML, O.Q6_K, O.Q6_K_GGML])
def test_gemv_brute_force_tiny(fmt):
    k = O.BLOCK_ELEMS[fmt] * 2
    n, b = 5, 3
    w = O.gen_weights(fmt, n, k, seed=fmt)
    x = O.gen_x(b, k, seed=1)
    W = O.dequant(fmt, w).reshape(n, k).astype(np.float64)
    want = (x.astype(np.float64) @ W.T).astype(np.float32)
    assert np.array_equal(O.gemv(fmt, w, x, n, k), want)
    # one-hot column selection
    xe = np.zeros((1, k), np.float32)
    xe[0, 3] = 1.0
    assert np.array_equal(O.gemv(fmt, w, xe, n, k)[0], W[:, 3].astype(np.float32))


def test_gemv_is_ref_gemm_with_transposed_weights():
    w = O.gen_weights(O.Q4_0, 6, 64, seed=9)
    x = O.gen_x(2, 64, seed=8)
    W = O.dequant(O.Q4_0, w).reshape(6, 64)
    assert np.array_equal(O.gemv(O.Q4_0, w, x, 6, 64), O.gemm_ref(x, W.T.copy()))


# ---- reference requant / layout helpers ------------------------------------------
def test_requant_int8_invariants():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal(32 * 50) * 0.1).astype(np.float32)
    w[:32] = 0.0
    q, s = O.requant_int8(w)
    assert np.abs(q.astype(int)).max() <= 127
    assert s[0] == 0 and np.all(q[:32] == 0)
    recon = q.astype(np.float32).reshape(-1, 32) * s[:, None]
    assert np.all(np.abs(recon - w.reshape(-1, 32)) <= s[:, None] / 2 * (1 + 1e-5) + 1e-12)
    assert np.allclose(s, np.abs(w.reshape(-1, 32)).max(1) / 127, rtol=1e-6)


def test_requant_int4_invariants_and_packing():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal(32 * 40) * 0.1).astype(np.float32)
    p, s = O.requant_int4(w)
    lo = (p & 15).astype(np.int8)
    hi = (p >> 4).astype(np.int8)
    lo = np.where(lo >= 8, lo - 16, lo)
    hi = np.where(hi >= 8, hi - 16, hi)
    q = np.empty(w.size, np.int8)
    q[0::2], q[1::2] = lo, hi  # even index in the low nibble
    assert q.min() >= -8 and q.max() <= 7
    recon = q.astype(np.float32).reshape(-1, 32) * s[:, None]
    assert np.all(np.abs(recon - w.reshape(-1, 32)) <= s[:, None] / 2 * (1 + 1e-5) + 1e-12)


def test_head_scales_and_gqa_transpose():
    rng = np.random.default_rng(5)
    D, kv, hd = 16, 8, 4
    w = rng.standard_normal(kv * D).astype(np.float32)
    hs = O.head_scales(w, kv // hd, hd, D)
    assert np.allclose(hs, np.abs(w.reshape(kv // hd, -1)).max(1))
    t = O.gqa_transpose(w, D, kv)
    assert np.array_equal(t.reshape(kv, D), w.reshape(D, kv).T)


def test_reference_int_wt_math():
    rng = np.random.default_rng(6)
    m, n, k = 3, 8, 64
    wf = rng.standard_normal((n, k)).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    q, s = O.requant_int8(wf)
    W = (q.astype(np.float32).reshape(-1, 32) * s[:, None]).reshape(n, k)
    assert np.array_equal(O.gemm_int8_wt(x, q, s, m, n, k), (x.astype(np.float64) @ W.T.astype(np.float64)).astype(np.float32))


def test_reference_launcher_scale_index_known_answer():
    """K % group_size != 0: the reference's GEMV kernels pick scale
    s_row[k/gs] with s_row = scales + (n*K)/gs (gemm_kernels.hip:610,615,
    781,796-797), its MFMA kernels scales[(n*K + k)/gs] (:717, :886).  Row 1
    of a K = 48, gs = 32 tensor starts at flat element 48: scale index 1.  For
    k = 20 the GEMV form gives 1 + 20 // 32 = 1, the flat form (48 + 20) // 32
    = 2; for k = 40: 1 + 1 = 2 and 88 // 32 = 2; for k = 10: 1 and 1."""
    n, k, gs = 2, 48, 32
    s = np.array([1.0, 10.0, 100.0, 1000.0], dtype=np.float32)  # ceil(96 / 32) = 3 used
    q8 = np.ones((n, k), dtype=np.int8)
    p4 = np.full(n * k // 2, 0x11, dtype=np.uint8)  # both nibbles = 1
    for col, gemv_scale, mfma_scale in ((20, 10.0, 100.0), (40, 100.0, 100.0), (10, 10.0, 10.0)):
        x = np.zeros((1, k), dtype=np.float32)
        x[0, col] = 1.0
        for route, want in ((True, gemv_scale), (False, mfma_scale)):
            y8 = O.gemm_int8_wt(x, q8, s, 1, n, k, gs, gemv_route=route)
            y4 = O.gemm_int4_wt(x, p4, s, None, 1, n, k, gs, 0, gemv_route=route)
            assert y8[0, 1] == want and y4[0, 1] == want, (col, route)
    # row 0 starts at 0: both forms agree
    x = np.zeros((1, k), dtype=np.float32)
    x[0, 40] = 1.0
    assert O.gemm_int8_wt(x, q8, s, 1, n, k, gs, gemv_route=True)[0, 0] == 10.0
    assert O.gemm_int8_wt(x, q8, s, 1, n, k, gs, gemv_route=False)[0, 0] == 10.0
    # the default route follows the reference launchers' M <= 32 switch
    x33 = np.zeros((33, k), dtype=np.float32)
    x33[:, 20] = 1.0
    assert O.gemm_int8_wt(x33, q8, s, 33, n, k, gs)[0, 1] == 100.0
    assert O.gemm_int8_wt(x33[:32], q8, s, 32, n, k, gs)[0, 1] == 10.0


def test_act_q8_quant_and_int_gemm():
    rng = np.random.default_rng(7)
    a = rng.standard_normal((4, 64)).astype(np.float32)
    q, d = O.quantize_act_q8(a)
    assert np.abs(q.astype(int)).max() <= 127
    w = O.gen_weights(O.Q8_0, 5, 64, seed=2)
    c = O.gemm_q8_i8(w, q, d, 5)
    blocks = w.reshape(5, 2, 34)
    dw = blocks[:, :, 0:2].copy().view(np.float16).astype(np.float64)[..., 0]
    qw = blocks[:, :, 2:].view(np.int8).astype(np.int64)
    qa = q.reshape(4, 2, 32).astype(np.int64)
    want = np.einsum("mbk,nbk,mb,nb->mn", qa, qw, d.astype(np.float64), dw)
    assert np.allclose(c, want, rtol=1e-6)


def _f32_samples(seed=7, n=200000):
    rng = np.random.default_rng(seed)
    bits = rng.integers(0, 2**32, size=n, dtype=np.uint64).astype(np.uint32)
    special = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0x33800000, 0x387FC000, 0x38800000,
                        0x477FE000, 0x477FF000, 0x47800000, 0x3F800000, 0x3F801000, 0xBF801FFF, 0x00000001],
                       dtype=np.uint32)
    normal = (rng.standard_normal(n) * 0.05).astype(np.float32).view(np.uint32)
    return np.concatenate([special, bits, normal]).view(np.float32)


def test_fp32_to_fp16_trunc_closed_form():
    """Truncating conversion (weight_loader.cpp:112-123): exact fp16 values
    round-trip; mantissa bits below fp16 precision are dropped (toward zero);
    below the fp16 normal range -> signed zero; at/above 2^16 -> signed Inf."""
    h = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    exp = (h >> 10) & 0x1F
    normal = (exp > 0) & (exp < 31)
    f = h[normal].view(np.float16).astype(np.float32)
    assert (O.fp32_to_fp16_trunc(f) == h[normal]).all()
    # an fp32 value strictly between two fp16 neighbours truncates to the lower magnitude
    nxt = np.nextafter(f, np.float32(np.inf) * np.sign(f)).astype(np.float32)
    assert (O.fp32_to_fp16_trunc(nxt) == h[normal]).all()
    t = O.fp32_to_fp16_trunc(np.array([1e-5, -1e-5, 6.1035156e-05, 65536.0, -1e9, np.inf, np.nan], np.float32))
    assert list(t) == [0x0000, 0x8000, 0x0400, 0x7C00, 0xFC00, 0x7C00, 0x7C00]


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
def test_fp32_to_fp16_trunc_matches_reference():
    R = O.ref()
    f = _f32_samples()
    ours = O.fp32_to_fp16_trunc(f)
    idx = np.random.default_rng(1).choice(f.size, 20000, replace=False)
    idx = np.concatenate([np.arange(15), idx])
    ref = np.array([R.gqref_fp32_to_fp16(float(v)) for v in f[idx]], dtype=np.uint16)
    assert (ours[idx] == ref).all()


def test_fp16_array_form_matches_scalar():
    h = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    a = O.fp16_to_fp32(h)
    L = O.lib()
    for v in range(0, 1 << 16, 97):
        assert a[v].tobytes() == np.float32(L.gqo_fp16_to_fp32(v)).tobytes()


def test_rmsnorm_closed_forms():
    K = 64
    gamma = np.linspace(0.5, 2.0, K).astype(np.float32)
    # constant row c: mean square c^2, normalised value c / sqrt(c^2 + eps)
    for c in (1.0, -3.0, 1e-3):
        x = np.full((1, K), c, dtype=np.float32)
        out = O.rmsnorm(x, gamma, 1e-5)
        ref = np.float64(np.float32(c)) / np.sqrt(np.float64(np.float32(c)) ** 2 + np.float64(np.float32(1e-5)))
        assert np.allclose(out[0], ref * gamma.astype(np.float64), rtol=1e-12, atol=0)
    # one-hot row: mean square 1/K
    x = np.zeros((2, K), dtype=np.float32)
    x[0, 5] = 2.0
    x[1, 0] = -1.0
    out = O.rmsnorm(x, np.ones(K, np.float32), 0.0)
    assert np.isclose(out[0, 5], np.sqrt(K)) and np.isclose(out[1, 0], -np.sqrt(K))
    assert np.count_nonzero(out) == 2
    # scale invariance: rmsnorm(a x) == rmsnorm(x) for eps = 0
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, K)).astype(np.float32)
    assert np.allclose(O.rmsnorm(x * 4, gamma, 0.0), O.rmsnorm(x, gamma, 0.0), rtol=1e-12)


def test_swiglu_closed_forms():
    g = np.array([0.0, 40.0, -40.0, 1.0, -1.0])
    u = np.array([3.0, 2.0, 5.0, 1.0, 1.0])
    out = O.swiglu(g, u)
    assert out[0] == 0.0
    assert np.isclose(out[1], 80.0) and abs(out[2]) < 1e-15
    # silu(1) - silu(-1) = 1 (silu(x) - silu(-x) = x)
    assert np.isclose(out[3] - out[4], 1.0, rtol=1e-15)
