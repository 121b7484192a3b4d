"""The C++ host mirror (GGUFLoader + GretaCompute::gemm, the reference's
interfaces) driven end to end by tests/cpp/greta_compute_driver.cpp on the GPU,
checked against the oracle within rel-L2 1e-3 (fp64-accumulated reference)."""
import os
import subprocess

import numpy as np
import pytest

import gguf_writer as W
import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DRIVER = os.path.join(ROOT, "gretacore-v3_amd", "lib", "greta_compute_driver")
TOL = 1e-3
DIM, HEADS, HEADS_KV, HD = 256, 4, 2, 64
KV = HEADS_KV * HD

TENSORS = [  # name, shape (ne0 first), ggml type, oracle fmt
    ("blk.0.ffn_gate.weight", [DIM, 512], W.GGML_Q4_0, O.Q4_0),
    ("blk.0.ffn_down.weight", [512, DIM], W.GGML_Q8_0, O.Q8_0),
    ("blk.0.attn_q.weight", [DIM, DIM], W.GGML_Q4_K, O.Q4_K),
    ("blk.0.attn_k.weight", [DIM, KV], W.GGML_Q4_K, O.Q4_K),
    ("output.weight", [DIM, 96], W.GGML_Q6_K, O.Q6_K),
]


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    d = tmp_path_factory.mktemp("mirror")
    path = str(d / "m.gguf")
    tensors, spec = [], {}
    for i, (nm, sh, gt, fmt) in enumerate(TENSORS):
        data = O.gen_weights(fmt, int(np.prod(sh)) // sh[0], sh[0], 300 + i).tobytes()
        tensors.append((nm, sh, gt, data))
        spec[nm] = (sh, fmt, np.frombuffer(data, dtype=np.uint8))
    W.write_gguf(path, W.llama_kv(dim=DIM, heads=HEADS, heads_kv=HEADS_KV), tensors)
    return path, spec, d


def _run(model, name, kind, M, label="", adt="f32", seed=0, path=None, a=None):
    gguf_path, spec, d = model
    path = path or gguf_path
    sh = spec[name][0]
    K = sh[0]
    N = int(np.prod(sh)) // K
    if a is None:
        a = O.gen_x(M, K, seed)
    ap, cp = str(d / f"a_{name}_{M}.f32"), str(d / f"c_{name}_{M}.f32")
    a.tofile(ap)
    r = subprocess.run([DRIVER, path, name, kind, str(M), ap, cp, label, adt], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr + r.stdout
    c = np.fromfile(cp, dtype=np.float32).reshape(M, N)
    route = r.stdout.split("route=")[1].split()[0]
    return a, c, route, N, K


def _round_a(a, adt):
    import torch
    if adt == "f16":
        return a.astype(np.float16).astype(np.float32)
    if adt == "bf16":
        return torch.from_numpy(a).to(torch.bfloat16).float().numpy()
    return a


pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,adt", [(1, "f32"), (4, "f32"), (16, "f32"), (64, "f32"), (96, "bf16"), (80, "f16")])
@pytest.mark.parametrize("name", ["blk.0.ffn_gate.weight", "blk.0.ffn_down.weight", "blk.0.attn_q.weight"])
def test_gemm_gguf_native(dev, model, name, M, adt):
    a, c, route, N, K = _run(model, name, "quant", M, adt=adt, seed=M)
    assert route == ("GEMV" if M <= 16 else "GEMM")
    sh, fmt, raw = model[1][name]
    ref = O.gemv(fmt, raw, _round_a(a, adt), N, K)
    assert O.rel_l2(c, ref) <= TOL


@pytest.mark.parametrize("M", [3, 5, 8, 12, 16])
@pytest.mark.parametrize("name", ["blk.0.ffn_gate.weight", "blk.0.ffn_down.weight", "blk.0.attn_q.weight",
                                  "output.weight"])
def test_gemm_gguf_native_wide_range_f32(dev, model, name, M):
    """GretaCompute::gemm with fp32 A of M <= 16 rows (the batch GEMV) on
    activations beyond fp16's range: spikes of 1e5 and a row of ~1e-6.  The
    reference's launchers keep fp32 activations for these rows
    (gemm_kernels.hip:594-634, 749-753); here every row must be finite and
    within 1e-3 of the fp64 oracle."""
    sh, fmt, raw = model[1][name]
    K = sh[0]
    N = int(np.prod(sh)) // K
    rng = np.random.default_rng(M)
    a = rng.standard_normal((M, K)).astype(np.float32)
    pos = rng.integers(0, K, size=(M, 4))
    for m in range(M):
        a[m, pos[m]] = (rng.choice([-1.0, 1.0], size=4) * 1e5 * (1 + rng.random(4))).astype(np.float32)
    a[M - 1] = (rng.standard_normal(K) * 1e-6).astype(np.float32)
    a, c, route, N, K = _run(model, name, "quant", M, seed=M, a=a)
    assert route == "GEMV"
    ref = O.gemv(fmt, raw, a, N, K)
    assert np.isfinite(c).all()
    for m in range(M):
        assert O.rel_l2(c[m], ref[m]) <= TOL, m


@pytest.mark.parametrize("M", [1, 8, 40])
@pytest.mark.parametrize("name", ["blk.0.ffn_gate.weight", "blk.0.attn_k.weight", "output.weight"])
def test_gemm_fp16_weights(dev, model, name, M):
    """load_tensor_fp16 (GGUF blocks dequantized, then rounded to fp16 with the
    reference's truncating conversion; K/V tensors GQA-reordered) and
    GretaCompute::gemm on the FP16 B it returns: the reference's FP16 route
    (greta_compute_hip.cpp:361-371), VALU launcher up to 32 rows, MFMA
    launcher above, against the fp64 product of the same fp16 weights."""
    a, c, route, N, K = _run(model, name, "fp16", M, seed=90 + M)
    assert route == ("VALU" if M <= 32 else "MFMA")
    sh, fmt, raw = model[1][name]
    w = O.dequant(fmt, raw)
    if "attn_k" in name:
        w = O.gqa_transpose(w, DIM, KV)
    w16 = O.fp16_to_fp32(O.fp32_to_fp16_trunc(np.ascontiguousarray(w, dtype=np.float32).ravel()))
    ref = a.astype(np.float64) @ w16.reshape(N, K).astype(np.float64).T
    assert O.rel_l2(c, ref) <= TOL


@pytest.mark.parametrize("M", [1, 40])
def test_gemm_q6k_output(dev, model, M):
    """Q6_K output.weight through GretaCompute::gemm: GEMV up to 16 rows, the
    skinny GEMM above (fp32 A)."""
    a, c, route, N, K = _run(model, "output.weight", "quant", M, seed=70 + M)
    assert route == ("GEMV" if M <= 16 else "GEMM")
    sh, fmt, raw = model[1]["output.weight"]
    assert O.rel_l2(c, O.gemv(fmt, raw, a, N, K)) <= TOL


@pytest.mark.parametrize("M", [1, 8, 33, 64])
@pytest.mark.parametrize("name", ["blk.0.attn_q.weight", "blk.0.attn_k.weight", "output.weight"])
@pytest.mark.parametrize("kind", ["int8", "int4"])
def test_gemm_reference_formats(dev, model, name, kind, M):
    """load_tensor_int8 / load_tensor_int4 (with GQA transpose and per-head
    scales) then GretaCompute::gemm -> the reference launchers' math."""
    a, c, route, N, K = _run(model, name, kind, M, seed=7 + M)
    assert route == ("GEMV" if M <= 32 else "GEMM")
    sh, fmt, raw = model[1][name]
    w = O.dequant(fmt, raw)
    if "attn_k" in name:
        w = O.gqa_transpose(w, DIM, KV)
    if kind == "int8":
        q, s = O.requant_int8(w)
        ref = O.gemm_int8_wt(a, q, s, M, N, K)
    else:
        q, s = O.requant_int4(w)
        hs = None
        if "attn_q" in name or "attn_k" in name:
            nh = HEADS_KV if "attn_k" in name else HEADS
            hs = O.head_scales(w, nh, HD, DIM)
        ref = O.gemm_int4_wt(a, q, s, hs, M, N, K, head_dim=(N // nh) if hs is not None else 0)
    assert O.rel_l2(c, ref) <= TOL


def test_int4_force_gemv_label(dev, model, monkeypatch):
    monkeypatch.setenv("GRETA_WO_LAYOUT_FORCE", "row")
    a, c, route, N, K = _run(model, "blk.0.attn_q.weight", "int4", 64, label="attn_o_prefill", seed=3)
    assert route == "GEMV"


@pytest.mark.parametrize("M", [1, 40])
@pytest.mark.parametrize("name", ["blk.0.ffn_gate.weight", "blk.0.attn_q.weight", "output.weight"])
def test_gemm_from_greta_cache(dev, model, name, M):
    """create_weight_loader on a .greta T16 cache -> GretaLoader::load_tensor_quant
    -> GretaCompute::gemm: the same result as from the GGUF."""
    import gq
    gguf_path, spec, d = model
    cache = str(d / "m.greta")
    if not os.path.exists(cache):
        with gq.GGUF(gguf_path) as g:
            gq.greta_write(g, cache, gq.LOAD_QUANT)
    a, c, route, N, K = _run(model, name, "quant", M, seed=50 + M, path=cache)
    _, c_gguf, route2, _, _ = _run(model, name, "quant", M, seed=50 + M)
    assert route == route2
    assert np.array_equal(c.view(np.uint32), c_gguf.view(np.uint32))


def test_int4_from_reference_format_greta(dev, model):
    """An INT4 .greta file (the reference tool's records) through
    GretaLoader::load_tensor_int4 -> GretaCompute::gemm equals the GGUF INT4 load."""
    import gq
    gguf_path, spec, d = model
    cache = str(d / "m_int4.greta")
    with gq.GGUF(gguf_path) as g:
        gq.greta_write(g, cache, gq.LOAD_INT4)
    for name in ("blk.0.attn_q.weight", "blk.0.attn_k.weight"):
        a, c, route, N, K = _run(model, name, "int4", 8, seed=5, path=cache)
        _, c_gguf, _, _, _ = _run(model, name, "int4", 8, seed=5)
        assert np.array_equal(c.view(np.uint32), c_gguf.view(np.uint32)), name
