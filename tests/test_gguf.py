"""GGUF loader: the build's parser and device loads (libgq.so, include/gq_gguf.h)
against the reference's own GGUFLoader (compiled into oracle/_ref from the
reference sources) and the oracle.

Files are written by tests/gguf_writer.py.  Parsing needs no GPU; the load
tests are marked gpu.  Reference quirks kept (weight_loader.cpp): data section
at the next 32-byte boundary; llama.* defaults from ModelConfig::llama2_7b;
GQA K/V tensors of shape [D, KV] transposed as if stored [D][KV].
Deliberate differences: Q8_0 is named "Q8_0" (the reference says "UNKNOWN"),
and 64-bit integer llama.* values are accepted."""
import os

import numpy as np
import pytest

import gguf_writer as W
import oracle as O

DIM, HEADS, HEADS_KV, HD = 256, 4, 2, 64
KV = HEADS_KV * HD
VOCAB = ["<unk>", "<s>", "</s>", "hello", "world", "x" * 2000, "end"]

# (name, shape (ne0 first), ggml type, oracle format)
TENSORS = [
    ("token_embd.weight", [DIM, 64], W.GGML_Q4_K, O.Q4_K),
    ("blk.0.attn_norm.weight", [DIM], W.GGML_F32, None),
    ("blk.0.attn_q.weight", [DIM, DIM], W.GGML_Q4_K, O.Q4_K),
    ("blk.0.attn_k.weight", [DIM, KV], W.GGML_Q4_K, O.Q4_K),
    ("blk.0.attn_v.weight", [DIM, KV], W.GGML_Q6_K, O.Q6_K),
    ("blk.0.attn_output.weight", [DIM, DIM], W.GGML_F16, None),
    ("blk.0.ffn_gate.weight", [DIM, 512], W.GGML_Q4_0, O.Q4_0),
    ("blk.0.ffn_down.weight", [512, DIM], W.GGML_Q8_0, O.Q8_0),
    ("blk.1.attn_k.weight", [KV, DIM], W.GGML_F16, None),
    ("blk.1.attn_v.weight", [DIM, KV], W.GGML_F32, None),
    ("output.weight", [DIM, 48], W.GGML_Q6_K, O.Q6_K),
]


def _tensor_data(name, shape, gt, fmt, seed):
    n = int(np.prod(shape))
    rng = np.random.default_rng(seed)
    if gt == W.GGML_F32:
        return (rng.standard_normal(n) * 0.05).astype(np.float32).tobytes()
    if gt == W.GGML_F16:
        return (rng.standard_normal(n) * 0.05).astype(np.float16).tobytes()
    rows = n // shape[0]
    return O.gen_weights(fmt, rows, shape[0], seed).tobytes()


@pytest.fixture(scope="module")
def model_file(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("gguf") / "tiny-llama.gguf")
    tensors = [(nm, sh, gt, _tensor_data(nm, sh, gt, f, 100 + i)) for i, (nm, sh, gt, f) in enumerate(TENSORS)]
    W.write_gguf(path, W.llama_kv(dim=DIM, heads=HEADS, heads_kv=HEADS_KV, layers=2, ff=512, ctx=2048,
                                  vocab=VOCAB, rope=500000.0, eps=1e-6), tensors)
    return path, {nm: (sh, gt, f, data) for nm, sh, gt, f, data in
                  [(t[0], t[1], t[2], TENSORS[i][3], t[3]) for i, t in enumerate(tensors)]}


def _ours(path):
    import gq
    return gq.GGUF(path)


# ---- parsing (CPU) -----------------------------------------------------------
def test_parse_matches_written_file(model_file):
    path, spec = model_file
    with _ours(path) as g:
        ts = g.tensors()
        assert [t["name"] for t in ts] == [t[0] for t in TENSORS]
        raw = open(path, "rb").read()
        for t in ts:
            sh, gt, fmt, data = spec[t["name"]]
            assert t["shape"] == sh and t["ggml_type"] == gt
            assert t["size_bytes"] == W.tensor_bytes(gt, sh) == len(data)
            assert t["offset"] % 32 == 0
            assert raw[t["offset"]:t["offset"] + t["size_bytes"]] == data
            assert g.read_raw(t["name"]).tobytes() == data
        c = g.config()
        assert (c["dim"], c["num_heads"], c["num_heads_kv"], c["head_dim"]) == (DIM, HEADS, HEADS_KV, HD)
        assert (c["num_layers"], c["hidden_dim"], c["max_seq_len"]) == (2, 512, 2048)
        assert c["rope_base"] == 500000.0 and c["rms_eps"] == np.float32(1e-6)
        assert c["vocab_size"] == len(VOCAB)
        voc = g.vocab()
        assert voc[:5] == [v.encode() for v in VOCAB[:5]]
        assert voc[5] == b"<too_long>" and voc[6] == b"end"


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
def test_parse_matches_reference_loader(model_file):
    path, _ = model_file
    rts, rcfg, err = O.ref_gguf_parse(path)
    assert rts is not None, err
    with _ours(path) as g:
        ts = g.tensors()
        assert len(ts) == len(rts)
        for a, b in zip(ts, rts):
            assert a["name"] == b["name"] and a["shape"] == b["shape"]
            assert a["offset"] == b["offset"] and a["size_bytes"] == b["size_bytes"]
            want = "UNKNOWN" if a["dtype"] == "Q8_0" else a["dtype"]
            assert want == b["dtype"]
        c = g.config()
        for k, v in rcfg.items():
            assert c[k] == v, k


def _write(tmp_path, name, kv, tensors, **kw):
    p = str(tmp_path / name)
    W.write_gguf(p, kv, tensors, **kw)
    return p


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
def test_defaults_and_key_order_match_reference(tmp_path):
    """No head_count_kv -> the 7B default (32) is kept; head_dim follows the
    last of embedding_length / head_count; other llama.* defaults stay."""
    kv = [("llama.attention.head_count", W.U32, 8), ("llama.embedding_length", W.I32, 512),
          ("llama.rope.freq_base", W.F32, 1234.5), ("some.other", W.ARR, (W.ARR, [(W.U8, [1, 2]), (W.U8, [3])])),
          ("llama.context_length", W.U16, 77)]
    data = O.gen_weights(O.Q4_0, 4, 64, 1).tobytes()
    p = _write(tmp_path, "d.gguf", kv[:3] + kv[4:], [("w", [64, 4], W.GGML_Q4_0, data)])
    rts, rcfg, err = O.ref_gguf_parse(p)
    assert rts is not None, err
    with _ours(p) as g:
        c = g.config()
        for k, v in rcfg.items():
            assert c[k] == v, k
        assert c["num_heads_kv"] == 32 and c["head_dim"] == 64 and c["max_seq_len"] == 77
        assert c["vocab_size"] == 32000 and c["num_layers"] == 32
    # nested arrays are skipped by the spec-following parser
    p2 = _write(tmp_path, "n.gguf", kv, [("w", [64, 4], W.GGML_Q4_0, data)])
    with _ours(p2) as g:
        assert g.tensors()[0]["name"] == "w"


def test_rejects_malformed_files(tmp_path):
    import gq
    data = O.gen_weights(O.Q4_0, 4, 64, 1).tobytes()
    good = _write(tmp_path, "ok.gguf", W.llama_kv(), [("w", [64, 4], W.GGML_Q4_0, data)])
    raw = open(good, "rb").read()
    cases = {
        "magic": b"GGUX" + raw[4:],
        "version": raw[:4] + (1).to_bytes(4, "little") + raw[8:],
        "truncated_header": raw[:40],
        "empty": b"",
    }
    for name, blob in cases.items():
        p = str(tmp_path / f"bad_{name}.gguf")
        open(p, "wb").write(blob)
        with pytest.raises(gq.GQError):
            gq.GGUF(p)
    # too many key/value pairs (the reference stops at 2000)
    p = _write(tmp_path, "kv.gguf", W.llama_kv(), [("w", [64, 4], W.GGML_Q4_0, data)], kv_count=2001)
    with pytest.raises(gq.GQError):
        gq.GGUF(p)
    with pytest.raises(gq.GQError, match="Not GGUF"):
        gq.GGUF(str(tmp_path / "bad_magic.gguf"))
    with pytest.raises(gq.GQError, match="Old GGUF"):
        gq.GGUF(str(tmp_path / "bad_version.gguf"))


def test_tensor_data_outside_file_is_an_error(tmp_path):
    import gq
    data = O.gen_weights(O.Q4_0, 4, 64, 1).tobytes()
    p = _write(tmp_path, "cut.gguf", W.llama_kv(), [("w", [64, 4], W.GGML_Q4_0, data)])
    blob = open(p, "rb").read()
    open(p, "wb").write(blob[:-10])
    with gq.GGUF(p) as g:
        assert g.tensors()[0]["size_bytes"] == len(data)
        with pytest.raises(gq.GQError, match="outside the file"):
            g.read_raw("w")
        with pytest.raises(gq.GQError, match="outside the file"):
            g.plan("w", gq.LOAD_QUANT)


def test_plans(model_file):
    import gq
    path, spec = model_file
    with _ours(path) as g:
        p = g.plan("blk.0.attn_k.weight", gq.LOAD_INT4)
        assert p["transpose"] and p["is_qkv"] and p["has_head_scales"] and p["num_heads"] == HEADS_KV
        assert p["bytes"] == DIM * KV // 2 and p["scale_bytes"] == DIM * KV // 32 * 4
        p = g.plan("blk.1.attn_k.weight", gq.LOAD_F16)
        assert not p["transpose"] and p["bytes"] == DIM * KV * 2
        p = g.plan("blk.0.ffn_down.weight", gq.LOAD_INT8)
        assert not p["transpose"] and p["bytes"] == 512 * DIM
        p = g.plan("blk.0.ffn_gate.weight", gq.LOAD_QUANT)
        assert (p["fmt"], p["N"], p["K"], p["bytes"]) == (gq.FMT_Q4_0, 512, DIM, gq.packed_size(gq.FMT_Q4_0, 512, DIM))
        p = g.plan("output.weight", gq.LOAD_QUANT)  # Q6_K: T16 too
        assert (p["fmt"], p["N"], p["K"]) == (gq.FMT_Q6_K, 48, DIM)
        with pytest.raises(gq.GQError, match="Q4_0, Q8_0, Q4_K or Q6_K"):
            g.plan("blk.0.attn_output.weight", gq.LOAD_QUANT)  # F16
        with pytest.raises(gq.GQError, match="not found"):
            g.plan("nope", gq.LOAD_F32)


# ---- device loads (GPU) ------------------------------------------------------
def _f32_of(spec_entry):
    sh, gt, fmt, data = spec_entry
    if gt == W.GGML_F32:
        return np.frombuffer(data, dtype=np.float32).copy()
    if gt == W.GGML_F16:
        return O.fp16_to_fp32(np.frombuffer(data, dtype=np.uint16))
    return O.dequant(fmt, np.frombuffer(data, dtype=np.uint8))


def _is_kv_transposed(name, shape):
    return ("attn_k.weight" in name or "attn_v.weight" in name) and shape == [DIM, KV]


def _oracle_load(name, spec_entry, kind):
    sh = spec_entry[0]
    w = _f32_of(spec_entry)
    if kind == 0:
        return w.view(np.uint8), None, None
    if kind == 2 and spec_entry[1] == W.GGML_Q8_0:
        blk = np.frombuffer(spec_entry[3], dtype=np.uint8).reshape(-1, 34)
        q = blk[:, 2:].copy().reshape(-1)
        s = O.fp16_to_fp32(blk[:, :2].copy().view(np.uint16).ravel())
        return q, s, None
    if _is_kv_transposed(name, sh):
        w = O.gqa_transpose(w, DIM, KV)
    if kind == 1:
        if spec_entry[1] == W.GGML_F16:  # stored fp16 is kept as is (subnormals included)
            h = np.frombuffer(spec_entry[3], dtype=np.uint16)
            if _is_kv_transposed(name, sh):
                h = h.reshape(DIM, KV).T.copy()
            return h.view(np.uint8), None, None
        return O.fp32_to_fp16_trunc(w).view(np.uint8), None, None
    if kind == 2:
        q, s = O.requant_int8(w)
        return q.view(np.uint8), s, None
    q, s = O.requant_int4(w)
    hs = None
    if any(t in name for t in ("attn_q", "attn_k", "attn_v")):
        nh = HEADS_KV if ("attn_k.weight" in name or "attn_v.weight" in name) else HEADS
        hs = O.head_scales(w, nh, HD, DIM)
    return q, s, hs


def _bits_equal(a, b):
    a = np.asarray(a).view(np.uint8).ravel()
    b = np.asarray(b).view(np.uint8).ravel()
    return a.size == b.size and bool((a == b).all())


REF_TYPES = (W.GGML_F32, W.GGML_F16, W.GGML_Q4_K, W.GGML_Q6_K)  # types the reference loader converts


@pytest.mark.gpu
@pytest.mark.parametrize("kind", [0, 1, 2, 3])
@pytest.mark.parametrize("name", [t[0] for t in TENSORS])
def test_load_matches_oracle(dev, model_file, name, kind):
    import gq
    path, spec = model_file
    with _ours(path) as g:
        data, sc, hs, plan = g.load(name, kind, device=dev)
    q, s, h = _oracle_load(name, spec[name], kind)
    assert _bits_equal(data.cpu().numpy(), q), name
    if s is not None:
        assert _bits_equal(sc.cpu().numpy(), s)
    if h is not None:
        assert _bits_equal(hs.cpu().numpy(), h)
    else:
        assert hs is None


@pytest.mark.gpu
@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("kind", [0, 1, 2, 3])
@pytest.mark.parametrize("name", [t[0] for t in TENSORS if t[2] in REF_TYPES])
def test_load_matches_reference_loader(dev, model_file, name, kind):
    """Bit-identical to the reference GGUFLoader run on the same file."""
    import gq
    path, spec = model_file
    rq, rs, rh = O.ref_gguf_load(path, name, kind, max_bytes=4 << 20)
    with _ours(path) as g:
        data, sc, hs, plan = g.load(name, kind, device=dev)
    assert _bits_equal(data.cpu().numpy(), rq), name
    if kind >= 2:
        assert _bits_equal(sc.cpu().numpy(), rs)
    if kind == 3 and rh.size:
        assert _bits_equal(hs.cpu().numpy(), rh)


@pytest.mark.gpu
@pytest.mark.parametrize("ggml", [False, True])
def test_load_quant_is_the_t16_repack(dev, model_file, ggml):
    import gq
    path, spec = model_file
    with _ours(path) as g:
        g.set_q4k_layout(ggml)
        for name, (sh, gt, fmt, data) in spec.items():
            if gt not in (W.GGML_Q4_0, W.GGML_Q8_0, W.GGML_Q4_K, W.GGML_Q6_K):
                continue
            packed, _, _, plan = g.load(name, gq.LOAD_QUANT, device=dev)
            f = plan["fmt"]
            if gt == W.GGML_Q4_K:
                assert f == (gq.FMT_Q4_K_GGML if ggml else gq.FMT_Q4_K)
            if gt == W.GGML_Q6_K:
                assert f == (gq.FMT_Q6_K_GGML if ggml else gq.FMT_Q6_K)
            k = sh[0]
            n = int(np.prod(sh)) // k
            host = gq.repack_host(f, np.frombuffer(data, dtype=np.uint8), n, k)
            assert _bits_equal(packed.cpu().numpy(), host), name
            # and the packed weights feed the GEMV directly
            x = O.gen_x(1, k, 5)
            import torch
            y = gq.gemv(f, packed, torch.from_numpy(x).to(dev), n, k).cpu().numpy()
            ref = O.gemv(f, np.frombuffer(data, dtype=np.uint8), x, n, k)
            assert O.rel_l2(y, ref) <= 1e-3


@pytest.mark.gpu
def test_sliced_upload_with_many_slices(dev, tmp_path, monkeypatch):
    """Tensors several times larger than the staging slice (1 MiB here, a ring
    of 2 slots) load bit-identically: every slot is reused, the last slice is
    short and the row count is not a multiple of 16."""
    import gq
    monkeypatch.setenv("GQ_LOAD_SLICE_MB", "1")
    monkeypatch.setenv("GQ_LOAD_SLOTS", "2")
    monkeypatch.setenv("GQ_LOAD_THREADS", "3")
    specs = [("a.weight", [4096, 1000], W.GGML_Q4_0, O.Q4_0), ("b.weight", [2048, 1000], W.GGML_Q6_K, O.Q6_K),
             ("c.weight", [1024, 900], W.GGML_Q8_0, O.Q8_0), ("d.weight", [3000, 700], W.GGML_F32, None),
             ("e.weight", [4096, 300], W.GGML_F16, None)]
    tensors = [(nm, sh, gt, _tensor_data(nm, sh, gt, f, 7 + i)) for i, (nm, sh, gt, f) in enumerate(specs)]
    path = _write(tmp_path, "big.gguf", W.llama_kv(dim=DIM, heads=HEADS, heads_kv=HEADS_KV, layers=1, ff=512,
                                                   ctx=2048, vocab=VOCAB, rope=1e4, eps=1e-5), tensors)
    with _ours(path) as g:
        for (nm, sh, gt, f), (_, _, _, data) in zip(specs, tensors):
            raw = np.frombuffer(data, dtype=np.uint8)
            k, n = sh[0], int(np.prod(sh)) // sh[0]
            if f is not None:
                packed, _, _, plan = g.load(nm, gq.LOAD_QUANT, device=dev)
                assert _bits_equal(packed.cpu().numpy(), gq.repack_host(f, raw, n, k)), nm
                f32, _, _, _ = g.load(nm, gq.LOAD_F32, device=dev)
                assert _bits_equal(f32.cpu().numpy(), O.dequant(f, raw)), nm
            elif gt == W.GGML_F32:
                f32, _, _, _ = g.load(nm, gq.LOAD_F32, device=dev)
                assert _bits_equal(f32.cpu().numpy(), raw), nm
            else:
                f16, _, _, _ = g.load(nm, gq.LOAD_F16, device=dev)
                assert _bits_equal(f16.cpu().numpy(), raw), nm
        q8, s8, _, _ = g.load("c.weight", gq.LOAD_INT8, device=dev)
        blk = np.frombuffer(tensors[2][3], dtype=np.uint8).reshape(-1, 34)  # Q8_0 split as stored
        assert _bits_equal(q8.cpu().numpy(), blk[:, 2:].copy())
        assert _bits_equal(s8.cpu().numpy(), O.fp16_to_fp32(blk[:, :2].copy().view(np.uint16).ravel()))


@pytest.mark.gpu
@pytest.mark.parametrize("slice_mb", ["1", "16"])
def test_load_quant_many_matches_single_loads(dev, tmp_path, monkeypatch, slice_mb):
    """gq_gguf_load_quant_many: several tensors of every quantized format,
    small and several slices long, ragged row counts, in one pipelined pass
    through a ring of 2 slots -- bit-identical to the host repack; the
    destinations of the failing calls (a missing name, a short destination,
    a non-quantized tensor) are checked before anything moves."""
    import torch

    import gq
    monkeypatch.setenv("GQ_LOAD_SLICE_MB", slice_mb)
    monkeypatch.setenv("GQ_LOAD_SLOTS", "2")
    specs = [("a.weight", [4096, 1000], W.GGML_Q4_0, O.Q4_0), ("b.weight", [2048, 333], W.GGML_Q6_K, O.Q6_K),
             ("c.weight", [1024, 900], W.GGML_Q8_0, O.Q8_0), ("d.weight", [512, 17], W.GGML_Q4_K, O.Q4_K),
             ("e.weight", [4096, 2000], W.GGML_Q4_K, O.Q4_K), ("f.weight", [64, 30], W.GGML_F32, None)]
    tensors = [(nm, sh, gt, _tensor_data(nm, sh, gt, f, 40 + i)) for i, (nm, sh, gt, f) in enumerate(specs)]
    path = _write(tmp_path, "many.gguf", W.llama_kv(dim=DIM, heads=HEADS, heads_kv=HEADS_KV, layers=1, ff=512,
                                                    ctx=2048, vocab=VOCAB, rope=1e4, eps=1e-5), tensors)
    quant = [(s, t) for s, t in zip(specs, tensors) if s[3] is not None]
    with _ours(path) as g:
        names = [s[0] for s, _ in quant] * 2  # each tensor twice: the ring wraps across tensors
        outs = [torch.full((g.plan(nm, gq.LOAD_QUANT)["bytes"],), 0xAB, dtype=torch.uint8, device=dev)
                for nm in names]
        g.load_quant_many(names, outs)
        for nm, o in zip(names, outs):
            (_, sh, _, f), (_, _, _, data) = next((s, t) for s, t in quant if s[0] == nm)
            k, n = sh[0], int(np.prod(sh)) // sh[0]
            assert _bits_equal(o.cpu().numpy(), gq.repack_host(f, np.frombuffer(data, dtype=np.uint8), n, k)), nm
        g.load_quant_many([], [])
        for bad_names, bad_outs in ((["a.weight", "nope.weight"], outs[:2]),
                                    (["a.weight", "c.weight"], [outs[0], outs[2][:-1]]),
                                    (["f.weight"], [torch.empty(64 * 30 * 4, dtype=torch.uint8, device=dev)])):
            before = [o.clone() for o in bad_outs]
            with pytest.raises(gq.GQError):
                g.load_quant_many(bad_names, bad_outs)
            for o, b in zip(bad_outs, before):
                assert torch.equal(o, b)


def _random_gguf(rng, path):
    """A GGUF file inside what the reference parser reads correctly: llama.*
    keys as integer / f32 scalars (not type 7, which it reads as a double),
    other keys of every scalar type, strings and flat arrays, a token list with
    over-long entries, and 1..10 tensors of every loader type."""
    u32_keys = ["llama.embedding_length", "llama.feed_forward_length", "llama.block_count",
                "llama.attention.head_count", "llama.attention.head_count_kv", "llama.context_length"]
    f32_keys = ["llama.rope.freq_base", "llama.norm_eps"]
    kv = []
    for key in u32_keys:
        if rng.random() < 0.85:
            t = int(rng.choice([W.U32, W.I32, W.U16, W.I16]))
            hi = {W.U32: 1 << 20, W.I32: 1 << 20, W.U16: 60000, W.I16: 30000}[t]
            kv.append((key, t, int(rng.integers(1, hi))))
    for key in f32_keys:
        if rng.random() < 0.85:
            kv.append((key, W.F32, float(np.float32(rng.uniform(1e-7, 1e6)))))
    scal = {W.U8: (0, 255), W.I8: (-128, 127), W.U16: (0, 65535), W.I16: (-32768, 32767), W.U32: (0, 1 << 31),
            W.I32: (-(1 << 31), 1 << 31), W.U64: (0, 1 << 62), W.I64: (-(1 << 62), 1 << 62)}
    for j in range(int(rng.integers(0, 8))):
        c = int(rng.integers(0, 5))
        key = f"general.extra_{j}"
        if c == 0:
            t = int(rng.choice(list(scal)))
            kv.append((key, t, int(rng.integers(*scal[t]))))
        elif c == 1:
            kv.append((key, int(rng.choice([W.F32, W.F64])), float(rng.standard_normal())))
        elif c == 2:
            kv.append((key, W.STR, "x" * int(rng.integers(0, 300))))
        elif c == 3:
            t = int(rng.choice(list(scal)))
            kv.append((key, W.ARR, (t, [int(v) for v in rng.integers(*scal[t], size=int(rng.integers(0, 40)))])))
        else:
            kv.append((key, W.ARR, (W.STR, ["s" * int(rng.integers(0, 20)) for _ in range(int(rng.integers(0, 30)))])))
    vocab = None
    if rng.random() < 0.7:
        vocab = ["t%d" % i if rng.random() < 0.95 else "L" * int(rng.integers(1025, 1500))
                 for i in range(int(rng.integers(1, 200)))]
        kv.append(("tokenizer.ggml.tokens", W.ARR, (W.STR, vocab)))
    order = rng.permutation(len(kv))
    kv = [kv[i] for i in order]
    types = [W.GGML_F32, W.GGML_F16, W.GGML_Q4_0, W.GGML_Q8_0, W.GGML_Q4_K, W.GGML_Q6_K]
    tensors = []
    for j in range(int(rng.integers(1, 11))):
        gt = int(rng.choice(types))
        be = W._BLOCK[gt][0]
        ne0 = be * int(rng.integers(1, 9)) if be > 1 else int(rng.integers(1, 600))
        shape = [ne0] + [int(rng.integers(1, 40)) for _ in range(int(rng.integers(0, 3)))]
        nb = W.tensor_bytes(gt, shape)
        tensors.append((f"blk.{j}.w{int(rng.integers(0, 1000))}.weight", shape, gt,
                        rng.integers(0, 256, nb, dtype=np.uint8).tobytes()))
    W.write_gguf(path, kv, tensors)
    return tensors, vocab


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
def test_parse_random_files_match_reference(tmp_path):
    """40 seeded random GGUF files: tensor tables, the config and the token
    list as the reference parser reads them (its Q8_0 dtype string is
    "UNKNOWN"), and every tensor's bytes where the file says they are."""
    rng = np.random.default_rng(20261205)
    for i in range(40):
        path = str(tmp_path / f"r{i}.gguf")
        tensors, vocab = _random_gguf(rng, path)
        rts, rcfg, err = O.ref_gguf_parse(path)
        assert rts is not None, (i, err)
        with _ours(path) as g:
            ts = g.tensors()
            assert len(ts) == len(rts) == len(tensors), i
            for a, b, (name, shape, gt, data) in zip(ts, rts, tensors):
                assert a["name"] == b["name"] == name and a["shape"] == b["shape"] == shape, i
                assert a["offset"] == b["offset"] and a["size_bytes"] == b["size_bytes"] == len(data), i
                assert ("UNKNOWN" if a["dtype"] == "Q8_0" else a["dtype"]) == b["dtype"], i
                assert g.read_raw(name).tobytes() == data, i
            c = g.config()
            for k, v in rcfg.items():
                assert c[k] == v, (i, k)
            if vocab is not None:
                assert g.vocab() == [b"<too_long>" if len(v) > 1024 else v.encode() for v in vocab], i


@pytest.mark.gpu
@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
def test_load_random_tensors_match_reference_loader(dev, tmp_path):
    """Random tensors of the types the reference loader converts (F32, F16,
    Q4_K, Q6_K; random ragged shapes, element counts a whole number of
    32-blocks) through every load kind (F32, F16, INT8, INT4), bit-identical to
    the reference GGUFLoader run on the same file.  Cases the reference
    refuses are skipped (none is expected)."""
    rng = np.random.default_rng(20261206)
    kinds_done = 0
    for f in range(6):
        tensors = []
        for j in range(6):
            gt = int(rng.choice([W.GGML_F32, W.GGML_F16, W.GGML_Q4_K, W.GGML_Q6_K]))
            be = W._BLOCK[gt][0]
            ne0 = be * int(rng.integers(1, 5)) if be > 1 else 32 * int(rng.integers(1, 40))
            shape = [ne0, int(rng.integers(1, 70))]
            tensors.append((f"blk.{j}.ffn_x{j}.weight", shape, gt,
                            _tensor_data(f"t{f}_{j}", shape, gt, O.Q4_K if gt == W.GGML_Q4_K else
                                         O.Q6_K if gt == W.GGML_Q6_K else None, 100 * f + j)))
        path = _write(tmp_path, f"rl{f}.gguf", W.llama_kv(dim=DIM, heads=HEADS, heads_kv=HEADS_KV, layers=1,
                                                          ff=512, ctx=2048, vocab=VOCAB, rope=1e4, eps=1e-5),
                      tensors)
        with _ours(path) as g:
            for name, shape, gt, _ in tensors:
                for kind in (0, 1, 2, 3):
                    print(f"random load file {f} {name} shape={shape} type={gt} kind={kind}", flush=True)
                    try:
                        rq, rs, rh = O.ref_gguf_load(path, name, kind, max_bytes=4 << 20)
                    except RuntimeError as e:
                        print("reference refused:", e, flush=True)
                        continue
                    data, sc, hs, _ = g.load(name, kind, device=dev)
                    assert _bits_equal(data.cpu().numpy(), rq), (name, kind)
                    if kind >= 2:
                        assert _bits_equal(sc.cpu().numpy(), rs), (name, kind)
                    kinds_done += 1
    assert kinds_done >= 100
