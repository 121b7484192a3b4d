"""GPU parity of the decode chain (gq_gemv_chain_*, include/gq_chain.h)
against the fp64 oracle: single GEMVs of every format and shape class
(ragged rows, fewer chunks than waves, K cut into column ranges), the
fused forms (RMSNorm, residual, GQA read, SwiGLU), a two-layer
Llama-3-8B-shaped decode step checked op by op, repeated runs and HIP graph
replays, and the bounded-wait error path."""
import os

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _w(fmt, n, k, seed, dev):
    import gq
    w = O.gen_weights(fmt, n, k, seed=seed)
    return w, gq.repack(fmt, _dev(w, dev), n, k)


@pytest.mark.parametrize("fmt", [O.Q4_0, O.Q8_0, O.Q4_K])
@pytest.mark.parametrize("n,k", [(4096, 4096), (1000, 512), (17, 256), (300, 14336), (4096, 2048), (300, 20480)])
def test_chain_single_gemv(dev, fmt, n, k):
    import torch

    import gq
    print(f"chain single fmt={fmt} n={n} k={k}", flush=True)
    w, p = _w(fmt, n, k, 10 + n, dev)
    x = O.gen_x(1, k, seed=20 + k)
    y = torch.full((n,), float("nan"), device=dev)
    ch = gq.Chain(fmt, [{"w": p, "x": _dev(x[0], dev), "y": y, "N": n, "K": k}], dev)
    ch.run()
    torch.cuda.synchronize()
    assert ch.error() == 0
    assert O.rel_l2(y.cpu().numpy(), O.gemv(fmt, w, x, n, k)[0]) <= TOL


def _gqa(v, heads, kv_heads, hd):
    """Attention over one cached position: query head h's output is v of kv
    head h // (heads / kv_heads)."""
    grp = heads // kv_heads
    return np.concatenate([v[(h // grp) * hd:(h // grp + 1) * hd] for h in range(heads)])


def _llama_layers(fmt, layers, dev, dim=4096, ff=14336, heads=32, kv=8, hd=128):
    import torch
    rng = np.random.default_rng(5)
    L = []
    for l in range(layers):
        mats = {}
        for nm, (n, k) in {"q": (dim, dim), "k": (kv * hd, dim), "v": (kv * hd, dim), "o": (dim, dim),
                           "g": (ff, dim), "u": (ff, dim), "d": (dim, ff)}.items():
            mats[nm] = _w(fmt, n, k, 100 * l + len(mats), dev)
        mats["an"] = (0.5 + rng.random(dim)).astype(np.float32)
        mats["fn"] = (0.5 + rng.random(dim)).astype(np.float32)
        L.append(mats)
    return L


def _decode_ops(L, h0, dev, dim=4096, ff=14336, kv=8, hd=128, grp=4):
    """The chain of a decode step: per layer q, k, v (RMSNorm fused), o
    (GQA read of v, residual), gate/up (RMSNorm, SwiGLU), down (residual)."""
    import torch
    bufs = {"h": [h0, torch.empty(dim, device=dev)], "h1": torch.empty(dim, device=dev),
            "q": torch.empty(dim, device=dev), "k": torch.empty(kv * hd, device=dev),
            "v": torch.empty(kv * hd, device=dev), "act": torch.empty(ff, device=dev)}
    ops, outs = [], []
    for l, m in enumerate(L):
        h_in, h_out = bufs["h"][l % 2], bufs["h"][(l + 1) % 2]
        an, fn = _dev(m["an"], dev), _dev(m["fn"], dev)
        m["_t"] = (an, fn)
        prev = [len(ops) - 1] if ops else []
        i0 = len(ops)
        ops.append({"w": m["q"][1], "x": h_in, "gamma": an, "y": bufs["q"], "N": dim, "K": dim, "deps": prev})
        ops.append({"w": m["k"][1], "x": h_in, "gamma": an, "y": bufs["k"], "N": kv * hd, "K": dim, "deps": prev})
        ops.append({"w": m["v"][1], "x": h_in, "gamma": an, "y": bufs["v"], "N": kv * hd, "K": dim, "deps": prev})
        ops.append({"w": m["o"][1], "x": bufs["v"], "x_head_dim": hd, "x_group": grp, "resid": h_in,
                    "y": bufs["h1"], "N": dim, "K": dim, "deps": [i0, i0 + 1, i0 + 2]})
        ops.append({"w": m["g"][1], "w_up": m["u"][1], "x": bufs["h1"], "gamma": fn, "y": bufs["act"],
                    "N": ff, "K": dim, "deps": [i0 + 3]})
        ops.append({"w": m["d"][1], "x": bufs["act"], "resid": bufs["h1"], "y": h_out, "N": dim, "K": ff,
                    "deps": [i0 + 4]})
    return ops, bufs


def _decode_ref(fmt, L, h, eps, dim=4096, ff=14336, heads=32, kv=8, hd=128):
    """The same step on the CPU: the fp64 oracle GEMVs, RMSNorm and SwiGLU."""
    steps = []
    for m in L:
        xn = O.rmsnorm(h[None], m["an"], eps)
        q = O.gemv(fmt, m["q"][0], xn, dim, dim)[0]
        v = O.gemv(fmt, m["v"][0], xn, kv * hd, dim)[0]
        h1 = h + O.gemv(fmt, m["o"][0], _gqa(v, heads, kv, hd)[None], dim, dim)[0]
        hn = O.rmsnorm(h1[None], m["fn"], eps)
        act = O.swiglu(O.gemv(fmt, m["g"][0], hn, ff, dim), O.gemv(fmt, m["u"][0], hn, ff, dim))[0]
        h = (h1 + O.gemv(fmt, m["d"][0], act[None], dim, ff)[0]).astype(np.float32)
        steps.append((q, v, h1, act, h))
    return steps


@pytest.mark.parametrize("fmt", [O.Q4_K, O.Q4_0, O.Q8_0])
def test_chain_llama_decode_two_layers(dev, fmt):
    import torch

    import gq
    print(f"chain llama 2 layers fmt={fmt}", flush=True)
    eps = 1e-5
    L = _llama_layers(fmt, 2, dev)
    h0 = O.gen_x(1, 4096, seed=3)[0] * 2.0
    ops, bufs = _decode_ops(L, _dev(h0, dev), dev)
    ch = gq.Chain(fmt, ops, dev, eps=eps)
    ref = _decode_ref(fmt, L, h0, eps)
    for rep in range(3):  # the counters are reset by every run
        bufs["h"][0].copy_(_dev(h0, dev))
        ch.run()
        torch.cuda.synchronize()
        assert ch.error() == 0
        assert O.rel_l2(bufs["h"][0].cpu().numpy(), ref[1][4]) <= TOL, rep
        # the last layer's intermediates
        q, v, h1, act, _ = ref[1]
        assert O.rel_l2(bufs["q"].cpu().numpy(), q) <= TOL
        assert O.rel_l2(bufs["v"].cpu().numpy(), v) <= TOL
        assert O.rel_l2(bufs["h1"].cpu().numpy(), h1) <= TOL
        assert O.rel_l2(bufs["act"].cpu().numpy(), act) <= TOL


@pytest.mark.parametrize("fmt", [O.Q4_0, O.Q4_K])
def test_chain_independent_stages(dev, fmt):
    """Ops that read different inputs and depend on nothing, interleaved with
    ops that share an input (one activation stage each run of them): every
    stage reuses the same LDS copy of x once the compute waves release it."""
    import torch

    import gq
    print(f"chain independent stages fmt={fmt}", flush=True)
    specs = [(512, 4096, 0), (256, 4096, 0), (2048, 1024, 1), (64, 14336, 2), (1024, 4096, 3), (1024, 4096, 3)]
    xs = {j: O.gen_x(1, k, seed=40 + j) for _, k, j in specs}
    ops, refs, ys = [], [], []
    for i, (n, k, j) in enumerate(specs):
        w, p = _w(fmt, n, k, 70 + i, dev)
        y = torch.full((n,), float("nan"), device=dev)
        ops.append({"w": p, "x": _dev(xs[j][0], dev), "y": y, "N": n, "K": k})
        refs.append(O.gemv(fmt, w, xs[j], n, k)[0])
        ys.append(y)
    ch = gq.Chain(fmt, ops, dev)
    for rep in range(2):
        ch.run()
        torch.cuda.synchronize()
        assert ch.error() == 0
        for i, (y, ref) in enumerate(zip(ys, refs)):
            assert O.rel_l2(y.cpu().numpy(), ref) <= TOL, (rep, i)


def test_chain_in_a_graph(dev):
    """A captured chain (fill kernel + one launch), replayed several times
    with eager work in between, matches the eager run every time."""
    import torch

    import gq
    print("chain graph replays", flush=True)
    fmt, eps = O.Q4_K, 1e-5
    L = _llama_layers(fmt, 1, dev)
    h0 = _dev(O.gen_x(1, 4096, seed=4)[0], dev)
    ops, bufs = _decode_ops(L, h0.clone(), dev)
    ch = gq.Chain(fmt, ops, dev, eps=eps)
    bufs["h"][0].copy_(h0)
    ch.run()
    torch.cuda.synchronize()
    eager = bufs["h"][1].clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            ch.run()
    torch.cuda.synchronize()
    for rep in range(4):
        bufs["h"][1].zero_()
        bufs["h"][0].copy_(h0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert ch.error() == 0
        assert torch.equal(bufs["h"][1], eager), rep


def test_chain_bounded_wait_drains(dev, monkeypatch):
    """A spin limit of 0 (forced from the host) makes any wait that finds its
    input unfinished give up at once: the launch still ends and the error flag
    is set -- with a layer's five dependent stages spread over every CU, the
    first poll of some workgroup always finds a producer unfinished -- and a
    plan with the normal limit then runs clean and gives the right output."""
    import torch

    import gq
    print("chain bounded wait", flush=True)
    fmt = O.Q4_K
    L = _llama_layers(fmt, 1, dev)
    h0 = _dev(O.gen_x(1, 4096, seed=6)[0], dev)
    ops, bufs = _decode_ops(L, h0.clone(), dev)
    monkeypatch.setenv("GQ_CHAIN_SPIN", "0")
    ch = gq.Chain(fmt, ops, dev)
    ch.run()
    torch.cuda.synchronize()
    assert ch.error() == 1
    monkeypatch.delenv("GQ_CHAIN_SPIN")
    ch2 = gq.Chain(fmt, ops, dev)
    bufs["h"][0].copy_(h0)
    ch2.run()
    torch.cuda.synchronize()
    assert ch2.error() == 0
    ref = _decode_ref(fmt, L, O.gen_x(1, 4096, seed=6)[0], 1e-5)
    assert O.rel_l2(bufs["h"][1].cpu().numpy(), ref[0][4]) <= TOL
