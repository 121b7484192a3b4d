""".greta files (include/gq_greta.h): the container of the reference's
pre-quantization tool (tools/quantize/greta_quantize_gguf.cpp:40-124) and the
T16 cache of the tiled layout.

The container is re-read here by an independent Python parser written from the
tool's write sequence (magic, json, count, then per tensor: name, dtype, rank,
u64 dims, group size, head count, three sizes, three arrays).  T16 records must
be gq_repack_host of the GGUF blocks; INT4 files must be, byte for byte, the file
the reference tool writes -- rebuilt here from the reference loader's own
load_tensor_int4 outputs (oracle/_ref) or, without it, from the oracle."""
import os
import struct

import numpy as np
import pytest

import gguf_writer as W
import oracle as O

DIM, HEADS, HEADS_KV, HD = 256, 4, 2, 64
KV = HEADS_KV * HD

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
    ("rope_freqs", [64], W.GGML_F32, None),  # no ".weight": never converted
    ("output.weight", [DIM, 48], W.GGML_Q6_K, O.Q6_K),
]
# the types the reference loader converts (its Q8_0 / Q4_0 handling differs, see test_gguf)
REF_TYPES = (W.GGML_F32, W.GGML_F16, W.GGML_Q4_K, W.GGML_Q6_K)


def _data(shape, gt, fmt, seed):
    n = int(np.prod(shape))
    rng = np.random.default_rng(seed)
    if gt == W.GGML_F32:
        return (rng.standard_normal(n) * 0.05).astype(np.float32).tobytes()
    if gt == W.GGML_F16:
        return (rng.standard_normal(n) * 0.05).astype(np.float16).tobytes()
    return O.gen_weights(fmt, n // shape[0], shape[0], seed).tobytes()


def _make(path, specs):
    tensors = [(nm, sh, gt, _data(sh, gt, f, 40 + i)) for i, (nm, sh, gt, f) in enumerate(specs)]
    W.write_gguf(path, W.llama_kv(dim=DIM, heads=HEADS, heads_kv=HEADS_KV, layers=1, ff=512, ctx=4096,
                                  vocab=["a", "b"], rope=500000.0, eps=1e-6), tensors)
    return {nm: (sh, gt, spec[3], d) for (nm, sh, gt, d), spec in zip(tensors, specs)}


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("greta") / "m.gguf")
    return path, _make(path, TENSORS)


def parse_container(blob: bytes):
    """Independent reader of the container: returns (json, [records])."""
    assert blob[:8] == b"GRETA_W\0"
    pos = 8
    (jl,) = struct.unpack_from("<I", blob, pos)
    js = blob[pos + 4:pos + 4 + jl].decode()
    pos += 4 + jl
    (n,) = struct.unpack_from("<I", blob, pos)
    pos += 4
    recs = []
    for _ in range(n):
        (nl,) = struct.unpack_from("<I", blob, pos)
        name = blob[pos + 4:pos + 4 + nl].decode()
        pos += 4 + nl
        dtype, rank = struct.unpack_from("<II", blob, pos)
        pos += 8
        dims = list(struct.unpack_from(f"<{rank}Q", blob, pos))
        pos += 8 * rank
        group, heads, ws, ss, hs = struct.unpack_from("<IIQQQ", blob, pos)
        pos += 32
        w = blob[pos:pos + ws]
        s = blob[pos + ws:pos + ws + ss]
        h = blob[pos + ws + ss:pos + ws + ss + hs]
        pos += ws + ss + hs
        recs.append({"name": name, "dtype": dtype, "dims": dims, "group": group, "heads": heads, "w": w, "s": s,
                     "h": h})
    assert pos == len(blob), "trailing bytes"
    return js, recs


def build_container(js: str, recs) -> bytes:
    """The reference tool's byte sequence for the given records."""
    out = [b"GRETA_W\0", struct.pack("<I", len(js)), js.encode(), struct.pack("<I", len(recs))]
    for r in recs:
        nm = r["name"].encode()
        out += [struct.pack("<I", len(nm)), nm, struct.pack("<II", r["dtype"], len(r["dims"])),
                struct.pack(f"<{len(r['dims'])}Q", *r["dims"]),
                struct.pack("<IIQQQ", r["group"], r["heads"], len(r["w"]), len(r["s"]), len(r["h"])),
                r["w"], r["s"], r["h"]]
    return b"".join(out)


T16_DTYPE = {O.Q4_0: 8, O.Q8_0: 9, O.Q4_K: 5, O.Q4_K_GGML: 10, O.Q6_K: 11, O.Q6_K_GGML: 12}


# ---- T16 files: written on the host, no GPU ----------------------------------
@pytest.mark.parametrize("ggml", [False, True])
def test_t16_file_holds_the_repacked_tiles(model, tmp_path, ggml):
    import gq
    path, spec = model
    out = str(tmp_path / "m.greta")
    with gq.GGUF(path) as g:
        g.set_q4k_layout(ggml)
        n = gq.greta_write(g, out, gq.LOAD_QUANT)
        cfg = g.config()
    js, recs = parse_container(open(out, "rb").read())
    assert not os.path.exists(out + ".tmp")
    want = [nm for nm, (sh, gt, f, d) in spec.items() if gt not in (W.GGML_F32, W.GGML_F16)]
    assert [r["name"] for r in recs] == want and n == len(want)
    for r in recs:
        sh, gt, f, d = spec[r["name"]]
        if ggml and f == O.Q4_K:
            f = O.Q4_K_GGML
        if ggml and f == O.Q6_K:
            f = O.Q6_K_GGML
        k, rows = sh[0], int(np.prod(sh)) // sh[0]
        assert r["dtype"] == T16_DTYPE[f] and r["dims"] == sh and r["heads"] == 0
        assert r["group"] == (32 if f in (O.Q4_0, O.Q8_0) else 256)
        assert r["s"] == b"" and r["h"] == b""
        assert r["w"] == gq.repack_host(f, np.frombuffer(d, dtype=np.uint8), rows, k).tobytes(), r["name"]
    assert '"layout": "t16"' in js and '"t16_version": 1' in js
    with gq.Greta(out) as h:
        assert h.config() == pytest.approx(cfg)
        ts = h.tensors()
        assert [t["name"] for t in ts] == want
        for t, r in zip(ts, recs):
            assert (t["dtype"], t["shape"], t["w_bytes"], t["s_bytes"]) == (r["dtype"], r["dims"], len(r["w"]), 0)
            assert t["fmt"] >= 0 and t["K"] == r["dims"][0] and t["N"] * t["K"] == int(np.prod(r["dims"]))


def test_reader_defaults_without_config(tmp_path):
    """A file with "{}" as json (what the reference tool writes) reads with the
    reference defaults (ModelConfig::llama2_7b)."""
    import gq
    p = str(tmp_path / "empty.greta")
    open(p, "wb").write(build_container("{}", []))
    with gq.Greta(p) as h:
        c = h.config()
        assert (c["dim"], c["num_heads"], c["num_layers"], c["vocab_size"], c["hidden_dim"]) == (4096, 32, 32, 32000,
                                                                                                  11008)
        assert h.tensors() == []


def _rec(name, dtype, dims, w, group=32, heads=0, s=b"", h=b""):
    return {"name": name, "dtype": dtype, "dims": dims, "group": group, "heads": heads, "w": w, "s": s, "h": h}


def test_reader_rejects_malformed_files(tmp_path):
    import gq
    good_w = gq.repack_host(O.Q4_0, O.gen_weights(O.Q4_0, 16, 64, 1), 16, 64).tobytes()
    js = '{"layout": "t16", "t16_version": 1}'
    ok = build_container(js, [_rec("a.weight", 8, [64, 16], good_w)])
    cases = {
        "magic": b"GRETA_X\0" + ok[8:],
        "truncated": ok[:-5],
        "count": ok[:8 + 4 + len(js)] + struct.pack("<I", 1 << 30) + ok[8 + 4 + len(js) + 4:],
        "version": build_container('{"layout": "t16", "t16_version": 99}', [_rec("a.weight", 8, [64, 16], good_w)]),
        "no version": build_container("{}", [_rec("a.weight", 8, [64, 16], good_w)]),
        "size": build_container(js, [_rec("a.weight", 8, [64, 16], good_w[:-1])]),
        "rank": build_container(js, [_rec("a.weight", 8, [64] * 9, good_w)]),
        "empty": b"",
    }
    for what, blob in cases.items():
        p = str(tmp_path / f"bad_{what.replace(' ', '_')}.greta")
        open(p, "wb").write(blob)
        with pytest.raises(gq.GQError):
            gq.Greta(p)
    p = str(tmp_path / "ok.greta")
    open(p, "wb").write(ok)
    with gq.Greta(p) as h:
        assert h.tensors()[0]["N"] == 16


def test_write_errors(model, tmp_path):
    import gq
    path, _ = model
    with gq.GGUF(path) as g:
        with pytest.raises(gq.GQError, match="cannot create"):
            gq.greta_write(g, str(tmp_path / "no" / "such" / "dir.greta"), gq.LOAD_QUANT)
        assert gq.load().gq_greta_write(g._h, str(tmp_path / "x.greta").encode(), gq.LOAD_F16, None) == 2


# ---- loads (GPU) -------------------------------------------------------------
@pytest.mark.gpu
def test_t16_load_equals_gguf_quant_load(dev, model, tmp_path):
    """Loading a tensor from the cache gives the bytes load_tensor_quant builds
    from the GGUF, and they feed the GEMV."""
    import gq
    import torch
    path, spec = model
    out = str(tmp_path / "m.greta")
    with gq.GGUF(path) as g:
        gq.greta_write(g, out, gq.LOAD_QUANT)
        with gq.Greta(out) as h:
            for t in h.tensors():
                w, s, hs = h.load(t["name"], device=dev)
                assert s is None and hs is None
                ref, _, _, plan = g.load(t["name"], gq.LOAD_QUANT, device=dev)
                assert torch.equal(w, ref), t["name"]
                x = O.gen_x(1, t["K"], 3)
                y = gq.gemv(t["fmt"], w, torch.from_numpy(x).to(dev), t["N"], t["K"]).cpu().numpy()
                raw = np.frombuffer(spec[t["name"]][3], dtype=np.uint8)
                assert O.rel_l2(y, O.gemv(t["fmt"], raw, x, t["N"], t["K"])) <= 1e-3


@pytest.mark.gpu
def test_int4_file_is_the_reference_tools_file(dev, tmp_path):
    """kind INT4 writes what tools/quantize/greta_quantize_gguf.cpp writes for
    the same GGUF: json "{}", every ".weight" tensor as load_tensor_int4's
    packed codes, scales and (attn_q/k/v) head scales."""
    import gq
    specs = [t for t in TENSORS if t[2] in REF_TYPES]
    path = str(tmp_path / "r.gguf")
    spec = _make(path, specs)
    out = str(tmp_path / "r.greta")
    with gq.GGUF(path) as g:
        n = gq.greta_write(g, out, gq.LOAD_INT4)
    recs = []
    for nm, sh, gt, f in specs:
        if ".weight" not in nm:
            continue
        if O.ref_available():
            q, s, h = O.ref_gguf_load(path, nm, 3, max_bytes=4 << 20)
        else:
            from test_gguf import _oracle_load
            q, s, h = _oracle_load(nm, spec[nm], 3)
            h = np.zeros(0, np.float32) if h is None else h
        qkv = any(t in nm for t in ("attn_q", "attn_k", "attn_v"))
        heads = (HEADS_KV if ("attn_k" in nm or "attn_v" in nm) else HEADS) if qkv else 0
        recs.append(_rec(nm, 4, sh, q.tobytes(), 32, heads, s.astype(np.float32).tobytes(),
                         h.astype(np.float32).tobytes()))
    assert n == len(recs)
    assert open(out, "rb").read() == build_container("{}", recs)
    # and the reader serves the records back
    with gq.Greta(out) as hd:
        for r in recs:
            w, s, h = hd.load(r["name"], device=dev)
            assert w.cpu().numpy().tobytes() == r["w"] and s.cpu().numpy().tobytes() == r["s"]
            assert (h.cpu().numpy().tobytes() if h is not None else b"") == r["h"]
