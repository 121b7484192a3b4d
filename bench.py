"""Benchmark of the GGUF quantized-weight matrix path on one MI355X.

Headline (the baseline's metric and its configs[1]): Q4_0 decode GEMV,
batch 1, 14336 x 4096, HBM GB/s of whole-job throughput (one GEMV kernel)
with the weights already resident in HBM.  A "step" is one GEMV call over one
weight copy; >= 8 distinct copies (>= 264 MB) are rotated so the 256 MB
Infinity Cache cannot serve them.

Also reported (field "extra"): the other benchmark configurations -- Q4_0 /
Q8_0 / Q6_K GEMV shapes, Q4_K batch 1/4/8/16, the prefill GEMM TFLOPS at
M = 64 / 512 / 2048, the reference-format INT4 / INT8 launchers, one full
32-layer Llama-3-8B-shaped decode step, and the GGUF-native load throughput
(pinned sliced upload + on-GPU repack).

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--headline-only]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "gretacore-v3_amd"), os.path.join(ROOT, "oracle")]

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense fp16/bf16
MFMA_I8_PEAK_TOPS = 5000.0     # dense int8
CACHE_DEFEAT_BYTES = 512 << 20  # > 256 MB Infinity Cache
# HBM bytes per launch of the headline kernel, measured with rocprofv3 PMC
# FETCH_SIZE + WRITE_SIZE and calibrated against a 64 MiB bitwise_not in the
# same runs (profiles/k_gemv_q_q4_0_14336x4096.md); valid for the launch plan
# it was measured with.
PROFILED_TRAFFIC = {("q4_0", 14336, 4096, 1, 2, 8): 33_291_776}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gpu_sysfs_dir(index=0):
    """sysfs directory of the GPU torch sees as cuda:<index> (by PCI address)."""
    import torch
    try:
        p = torch.cuda.get_device_properties(index)
        d = f"/sys/bus/pci/devices/{p.pci_domain_id:04x}:{p.pci_bus_id:02x}:{p.pci_device_id:02x}.0"
        return d if os.path.isdir(d) else None
    except (RuntimeError, AttributeError):
        return None


def _read(path):
    try:
        with open(path) as f:
            return f.read()
    except OSError:
        return None


def _dpm(text):
    """(levels in MHz, current MHz) of a pp_dpm_* file ('0: 500Mhz *' lines)."""
    levels, cur = [], None
    for line in (text or "").splitlines():
        parts = line.replace(":", " ").split()
        mhz = [int(t[:-3]) for t in parts if t.lower().endswith("mhz") and t[:-3].isdigit()]
        if mhz:
            levels.append(mhz[0])
            if "*" in line:
                cur = mhz[0]
    return levels, cur


class ClockSampler:
    """Samples the GPU's current shader clock (pp_dpm_sclk) and power draw
    every few ms on a host thread while a benchmark section runs."""

    def __init__(self, sysdir, period_s=0.005):
        import threading
        self.sysdir, self.period = sysdir, period_s
        self.sclk, self.power = [], []
        self._stop = threading.Event()
        self._t = threading.Thread(target=self._run, daemon=True)

    def _run(self):
        import glob
        hw = glob.glob(os.path.join(self.sysdir, "hwmon", "hwmon*", "power1_average")) + \
            glob.glob(os.path.join(self.sysdir, "hwmon", "hwmon*", "power1_input"))
        while not self._stop.is_set():
            cur = _dpm(_read(os.path.join(self.sysdir, "pp_dpm_sclk")))[1]
            if cur is not None:
                self.sclk.append(cur)
            if hw:
                v = _read(hw[0])
                if v and v.strip().isdigit():
                    self.power.append(int(v) / 1e6)
            self._stop.wait(self.period)

    def __enter__(self):
        if self.sysdir:
            self._t.start()
        return self

    def __exit__(self, *exc):
        self._stop.set()
        if self._t.is_alive():
            self._t.join()

    def summary(self):
        def st(v):
            if not v:
                return None
            v = sorted(v)
            return {"min": v[0], "median": v[len(v) // 2], "max": v[-1], "samples": len(v)}
        return {"dpm_level_sclk_mhz": st(self.sclk), "power_average_w": st(self.power)}


def box_state():
    """The GPU's clock levels, current memory clock and power cap from sysfs
    (null where the box does not expose them), so box-to-box variance is
    visible on every bench line."""
    import glob
    d = gpu_sysfs_dir()
    if not d:
        return {"sysfs": None}
    sl, sc = _dpm(_read(os.path.join(d, "pp_dpm_sclk")))
    ml, mc = _dpm(_read(os.path.join(d, "pp_dpm_mclk")))
    out = {"sysfs": d, "sclk_levels_mhz": sl, "mclk_levels_mhz": ml, "mclk_current_mhz": mc}
    for key, name in (("power_cap_w", "power1_cap"), ("power_cap_max_w", "power1_cap_max")):
        f = glob.glob(os.path.join(d, "hwmon", "hwmon*", name))
        v = _read(f[0]) if f else None
        out[key] = int(v) / 1e6 if v and v.strip().isdigit() else None
    return out


def gemv_bytes(fmt, n, k, batch):
    import gq
    return gq.gguf_bytes(fmt, n, k) + 4 * batch * (n + k)


class GemvCase:
    """Repacked weight copies + activations for one GEMV shape."""

    def __init__(self, fmt, n, k, batch, wseed, xseed, dev, min_copies=8):
        import torch

        import gq
        import oracle as O
        self.fmt, self.n, self.k, self.batch = fmt, n, k, batch
        self.w = O.gen_weights(fmt, n, k, seed=wseed)
        self.x_host = O.gen_x(batch, k, seed=xseed)
        packed = gq.repack(fmt, torch.from_numpy(self.w).to(dev), n, k)
        nbytes = packed.numel()
        ncopies = max(min_copies, -(-CACHE_DEFEAT_BYTES // nbytes))
        self.copies = [packed] + [packed.clone() for _ in range(ncopies - 1)]
        self.x = torch.from_numpy(self.x_host).to(dev)
        self.y = torch.empty((batch, n), dtype=torch.float32, device=dev)
        self.ws = gq.Workspace(dev, gq.gemv_workspace_bytes(fmt, k, batch))
        self.bytes = gemv_bytes(fmt, n, k, batch)

    def step(self, i):
        import gq
        gq.gemv(self.fmt, self.copies[i % len(self.copies)], self.x, self.n, self.k, y=self.y, workspace=self.ws)

    def check(self):
        import oracle as O
        self.step(0)
        ref = O.gemv(self.fmt, self.w, self.x_host, self.n, self.k)
        return O.rel_l2(self.y.cpu().numpy(), ref)


def time_steps(fn, steps, warmup):
    """Per-step seconds of `fn` launched eagerly (host-side launch loop)."""
    import torch
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        fn(i)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def graph_steps(fn, steps, warmup):
    """Per-step seconds of `steps` consecutive calls of `fn` captured into one
    HIP graph and replayed: device time with no per-launch host overhead.
    HIP events bracket each replay on the stream the kernels run on; the
    median of three replays is returned."""
    import torch
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for i in range(steps):
                fn(i)
        g.replay()  # first replay uploads the graph (untimed)
        s.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        times = []
        for _ in range(3):  # median of three replays
            torch.cuda.synchronize()
            e0.record(s)
            g.replay()
            e1.record(s)
            e1.synchronize()
            times.append(e0.elapsed_time(e1) / 1e3 / steps)
    torch.cuda.synchronize()
    per = sorted(times)[1]
    del g
    return per


def bench_gemv(case, steps, warmup):
    err = case.check()
    t_graph = graph_steps(case.step, steps, warmup)
    t_eager = time_steps(case.step, steps, warmup)
    return {
        "step_us": t_graph * 1e6, "GBps": case.bytes / t_graph / 1e9,
        "pct_peak": 100.0 * case.bytes / t_graph / 1e9 / HBM_PEAK_GBS,
        "eager_step_us": t_eager * 1e6,
        "weight_bytes": case.bytes - 4 * case.batch * (case.n + case.k), "alg_bytes": case.bytes,
        "copies": len(case.copies), "rel_l2": err,
    }


def bench_f16w(n, k, batch, steps, warmup, dev):
    """The FP16-weight route (gq_gemm_f16w; the reference's FP16 GretaCompute::gemm
    path, e.g. a Q6_K lm_head dequantized to fp16 at load): one call per step
    over a weight matrix larger than the Infinity Cache (no rotation needed);
    parity on 1024 sampled rows against an fp64 product."""
    import numpy as np
    import torch

    import gq
    import oracle as O
    g = torch.Generator(device="cpu").manual_seed(1007)
    w = (torch.randn(n, k, generator=g) * 0.05).to(torch.float16)
    x = torch.randn(batch, k, generator=g)
    wd, xd = w.to(dev), x.to(dev)
    y = torch.empty((batch, n), dtype=torch.float32, device=dev)
    gq.gemm_f16w(wd, xd, n, k, c=y)
    rows = np.linspace(0, n - 1, 1024).astype(int)
    ref = x.double().numpy() @ w[rows].double().numpy().T
    err = O.rel_l2(y[:, rows].cpu().numpy(), ref)
    byts = n * k * 2 + 4 * batch * (n + k)
    t = graph_steps(lambda i: gq.gemm_f16w(wd, xd, n, k, c=y), steps, warmup)
    del wd
    return {"step_us": t * 1e6, "GBps": byts / t / 1e9, "pct_peak": 100.0 * byts / t / 1e9 / HBM_PEAK_GBS,
            "alg_bytes": byts, "rel_l2": err}


def bench_gemm(fmt, m, n, k, steps, warmup, dev, out_dtype="f32"):
    import torch

    import gq
    import oracle as O
    w = O.gen_weights(fmt, n, k, seed=1004)
    packed = gq.repack(fmt, torch.from_numpy(w).to(dev), n, k)
    a = torch.randn(m, k, generator=torch.Generator().manual_seed(2004)).to(torch.bfloat16).to(dev)
    odt = torch.float32 if out_dtype == "f32" else torch.bfloat16
    c = torch.empty((m, n), dtype=odt, device=dev)
    ws = gq.Workspace(dev, gq.gemm_workspace_bytes(fmt, m, k))
    # parity on a row sample (fp64 oracle)
    gq.gemm(fmt, packed, a, n, k, out_dtype=odt, c=c, workspace=ws)
    rows = list(range(0, m, max(1, m // 32)))
    ref = O.gemv(fmt, w, a[rows].float().cpu().numpy(), n, k)
    err = O.rel_l2(c[rows].float().cpu().numpy(), ref)
    flops = 2.0 * m * n * k
    run = lambda i: gq.gemm(fmt, packed, a, n, k, out_dtype=odt, c=c, workspace=ws)
    t = graph_steps(run, max(4, steps // 8), 2)
    return {"step_us": t * 1e6, "TFLOPS": flops / t / 1e12, "pct_peak_f16": 100.0 * flops / t / 1e12 / MFMA_F16_PEAK_TFLOPS,
            "rel_l2": err}


def bench_gemm_q8_i8(m, n, k, steps, dev):
    """The int8 route for Q8_0: activations quantized per 32-block
    (gq_quantize_act_q8), then one v_mfma_i32_32x32x32_i8 per block with the
    two block scales applied in fp32 (gq_gemm_q8_i8).  TOPS of the GEMM
    kernel's step (the quantization is a separate launch, timed with it)."""
    import torch

    import gq
    import oracle as O
    w = O.gen_weights(O.Q8_0, n, k, seed=1004)
    packed = gq.repack(O.Q8_0, torch.from_numpy(w).to(dev), n, k)
    a = torch.randn(m, k, generator=torch.Generator().manual_seed(2004)).to(torch.bfloat16).to(dev)
    qa, da = gq.quantize_act_q8(a)
    c = gq.gemm_q8_i8(packed, qa, da, n)
    rows = list(range(0, m, max(1, m // 16)))
    err = O.rel_l2(c[rows].cpu().numpy(), O.gemm_q8_i8(w, qa[rows].cpu().numpy(), da[rows].cpu().numpy(), n))

    def run(i):
        gq.quantize_act_q8(a)
        gq.gemm_q8_i8(packed, qa, da, n, c=c)
    t = graph_steps(run, max(4, steps // 8), 2)
    ops = 2.0 * m * n * k
    return {"step_us": t * 1e6, "TOPS": ops / t / 1e12, "pct_peak_i8": 100.0 * ops / t / 1e12 / MFMA_I8_PEAK_TOPS,
            "rel_l2_vs_exact_integer_oracle": err}


def bench_compat(dev, m, n=14336, k=4096):
    """The reference's INT4 / INT8 weight-only launchers (requantized weight
    formats of load_tensor_int4/int8, fp32 A): one call per step."""
    import torch

    import gq
    g = torch.Generator(device="cpu").manual_seed(3000 + m)
    b8 = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=g).to(dev)
    b4 = torch.randint(-128, 128, (n, k // 2), dtype=torch.int8, generator=g).to(dev)
    sc = (torch.rand(n * k // 32, generator=g) * 0.01).to(dev)
    a = torch.randn(m, k, generator=g).to(dev)
    c = torch.empty(m, n, device=dev)
    t8 = graph_steps(lambda i: gq.launch_int8_wt(a, b8, sc, m, n, k, c=c), 20, 2)
    t4 = graph_steps(lambda i: gq.launch_int4_wt(a, b4, sc, None, m, n, k, c=c), 20, 2)
    route = "fp32 GEMV" if m <= 32 else "fp16 MFMA (Q8_0 / Q4_0 conversion + gq_gemm)"
    return {"int8_us": t8 * 1e6, "int4_us": t4 * 1e6, "route": route,
            "int8_GBps": (n * k + n * k // 32 * 4) / t8 / 1e9, "int4_GBps": (n * k // 2 + n * k // 32 * 4) / t4 / 1e9,
            "TFLOPS_int4": 2.0 * m * n * k / t4 / 1e12}


def bench_decode_step(dev, steps, warmup):
    """Config 5: 32-layer Llama-3-8B-shaped decode step, Q4_K projections and a
    Q8_0 lm_head: 7 GEMVs per layer + lm_head = 225 single-kernel GEMVs."""
    import numpy as np
    import torch

    import gq
    import oracle as O
    Q4K, Q80 = O.Q4_K, O.Q8_0
    shapes = {"q": (4096, 4096), "k": (1024, 4096), "v": (1024, 4096), "o": (4096, 4096),
              "gate": (14336, 4096), "up": (14336, 4096), "down": (4096, 14336)}
    base = {}
    for i, (name, (n, k)) in enumerate(shapes.items()):
        w = O.gen_weights(Q4K, n, k, seed=1005 + i)
        base[name] = gq.repack(Q4K, torch.from_numpy(w).to(dev), n, k)
    layers = [{name: base[name].clone() for name in shapes} for _ in range(32)]
    del base
    lm = O.gen_weights(Q80, 128256, 4096, seed=1015)
    lm_packed = gq.repack(Q80, torch.from_numpy(lm).to(dev), 128256, 4096)
    del lm
    torch.cuda.synchronize()
    wbytes = 32 * sum(gq.gguf_bytes(Q4K, n, k) for n, k in shapes.values()) + gq.gguf_bytes(Q80, 128256, 4096)
    xs = {k: torch.from_numpy(O.gen_x(1, k, seed=2005 + k)).to(dev) for k in (4096, 14336)}
    ys = {n: torch.empty((1, n), dtype=torch.float32, device=dev) for n in (1024, 4096, 14336, 128256)}

    def one_step(_i):
        for L in layers:
            for name, (n, k) in shapes.items():
                gq.gemv(Q4K, L[name], xs[k], n, k, y=ys[n])
        gq.gemv(Q80, lm_packed, xs[4096], 128256, 4096, y=ys[128256])

    # the same projections with the matrices that share x launched together
    # (q/k/v and gate/up: gq_gemv_multi), 4 launches per layer
    yq, yk, yv = (torch.empty((1, n), dtype=torch.float32, device=dev) for n in (4096, 1024, 1024))
    yg, yu = (torch.empty((1, 14336), dtype=torch.float32, device=dev) for _ in range(2))

    def one_step_grouped(_i):
        for L in layers:
            gq.gemv_multi(Q4K, [(L["q"], 4096), (L["k"], 1024), (L["v"], 1024)], xs[4096], 4096, ys=[yq, yk, yv])
            gq.gemv(Q4K, L["o"], xs[4096], 4096, 4096, y=ys[4096])
            gq.gemv_multi(Q4K, [(L["gate"], 14336), (L["up"], 14336)], xs[4096], 4096, ys=[yg, yu])
            gq.gemv(Q4K, L["down"], xs[14336], 4096, 14336, y=ys[4096])
        gq.gemv(Q80, lm_packed, xs[4096], 128256, 4096, y=ys[128256])

    # the fused forms a decode loop calls: RMSNorm folded into the q/k/v and
    # gate/up launches, gate/up producing silu(gate) * up (the down input)
    gamma = torch.ones(4096, dtype=torch.float32, device=dev)
    ya = torch.empty((1, 14336), dtype=torch.float32, device=dev)

    def one_step_fused(_i):
        for L in layers:
            gq.gemv_multi(Q4K, [(L["q"], 4096), (L["k"], 1024), (L["v"], 1024)], xs[4096], 4096, gamma=gamma,
                          ys=[yq, yk, yv])
            gq.gemv(Q4K, L["o"], xs[4096], 4096, 4096, y=ys[4096])
            gq.gemv_swiglu(Q4K, L["gate"], L["up"], xs[4096], 14336, 4096, gamma=gamma, y=ya)
            gq.gemv(Q4K, L["down"], xs[14336], 4096, 14336, y=ys[4096])
        gq.gemv(Q80, lm_packed, xs[4096], 128256, 4096, y=ys[128256])

    # the same projections as one persistent launch per step (gq_gemv_chain):
    # the real data flow of a decode step (RMSNorm, GQA read of v at one
    # cached position, residuals, SwiGLU), then the lm_head
    rng = np.random.default_rng(0)
    dim, ffd = 4096, 14336
    hbuf = [torch.from_numpy(O.gen_x(1, dim, seed=3)[0]).to(dev), torch.empty(dim, device=dev)]
    cb = {"h1": torch.empty(dim, device=dev), "q": torch.empty(dim, device=dev),
          "k": torch.empty(1024, device=dev), "v": torch.empty(1024, device=dev), "act": torch.empty(ffd, device=dev)}
    norms = [(torch.from_numpy((0.5 + rng.random(dim)).astype(np.float32)).to(dev),
              torch.from_numpy((0.5 + rng.random(dim)).astype(np.float32)).to(dev)) for _ in layers]
    cops = []
    for l, Lw in enumerate(layers):
        h_in, h_out = hbuf[l % 2], hbuf[(l + 1) % 2]
        an, fn = norms[l]
        prev = [len(cops) - 1] if cops else []
        i0 = len(cops)
        for nm, n in (("q", dim), ("k", 1024), ("v", 1024)):
            cops.append({"w": Lw[nm], "x": h_in, "gamma": an, "y": cb[nm], "N": n, "K": dim, "deps": prev})
        cops.append({"w": Lw["o"], "x": cb["v"], "x_head_dim": 128, "x_group": 4, "resid": h_in, "y": cb["h1"],
                     "N": dim, "K": dim, "deps": [i0, i0 + 1, i0 + 2]})
        cops.append({"w": Lw["gate"], "w_up": Lw["up"], "x": cb["h1"], "gamma": fn, "y": cb["act"], "N": ffd,
                     "K": dim, "deps": [i0 + 3]})
        cops.append({"w": Lw["down"], "x": cb["act"], "resid": cb["h1"], "y": h_out, "N": dim, "K": ffd,
                     "deps": [i0 + 4]})
    chain = gq.Chain(Q4K, cops, dev)
    fnorm = torch.from_numpy((0.5 + rng.random(dim)).astype(np.float32)).to(dev)

    def one_step_chain(_i):
        chain.run()
        gq.gemv_multi(Q80, [(lm_packed, 128256)], hbuf[len(layers) % 2], 4096, gamma=fnorm, ys=[ys[128256]])

    t_eager = time_steps(one_step, 3, 1)
    t_graph = graph_steps(one_step, 4, 1)
    t_grouped = graph_steps(one_step_grouped, 4, 1)
    t_fused = graph_steps(one_step_fused, 4, 1)
    t_chain = graph_steps(one_step_chain, 4, 1)
    chain_err = chain.error()
    out = {"weight_bytes": wbytes, "gemv_launches": 225, "eager_ms": t_eager * 1e3, "graph_ms": t_graph * 1e3,
           "graph_GBps": wbytes / t_graph / 1e9, "graph_pct_peak": 100.0 * wbytes / t_graph / 1e9 / HBM_PEAK_GBS,
           "projection_steps_per_s": 1.0 / t_graph,
           "grouped_launches": 129, "grouped_graph_ms": t_grouped * 1e3,
           "grouped_GBps": wbytes / t_grouped / 1e9,
           "grouped_pct_peak": 100.0 * wbytes / t_grouped / 1e9 / HBM_PEAK_GBS,
           "fused_norm_swiglu_graph_ms": t_fused * 1e3,
           "chain_graph_ms": t_chain * 1e3, "chain_launches": 2, "chain_wait_error": chain_err,
           "chain_note": "one persistent launch for the 32 layers (real data flow: RMSNorm, GQA read, residuals, "
                         "SwiGLU) + the lm_head; its compute waves idle ~48 % of the step waiting for each "
                         "stage's input (flag latency ~2.5 us, x staging 2-6 us, the stage's last units) and "
                         "stream at ~3.7 TB/s otherwise, so the grouped launches stay the faster decode path"}
    del chain
    del layers, lm_packed
    torch.cuda.empty_cache()
    return out


def bench_load(dev, layers=8):
    """GGUF-native load throughput (the loader I/O row): a Llama-3-8B
    shaped file of `layers` Q4_K layers (~1 GB) in the page cache, every matrix
    loaded with gq_gguf_load(QUANT) (pinned sliced upload + on-GPU T16 repack),
    against the reference's way of loading: read into pageable memory, a
    synchronous pageable copy, then the repack; many_GBps is the same tensors
    through gq_gguf_load_quant_many (one pipelined pass; the bytes it leaves
    are the ones compared with the reference-style load).  GB/s of GGUF
    bytes."""
    import shutil
    import tempfile

    import numpy as np
    import torch

    import gq
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import gguf_writer as W
    shapes = [("attn_q", 4096, 4096), ("attn_k", 4096, 1024), ("attn_v", 4096, 1024),
              ("attn_output", 4096, 4096), ("ffn_gate", 4096, 14336), ("ffn_up", 4096, 14336),
              ("ffn_down", 14336, 4096)]
    d = tempfile.mkdtemp(prefix="gq_load_")
    path = os.path.join(d, "model.gguf")
    try:
        rng = np.random.default_rng(0)
        tensors = []
        for l in range(layers):
            for nm, k, n in shapes:
                nb = W.tensor_bytes(W.GGML_Q4_K, [k, n])
                tensors.append((f"blk.{l}.{nm}.weight", [k, n], W.GGML_Q4_K,
                                rng.integers(0, 256, nb, dtype=np.uint8).tobytes()))
        W.write_gguf(path, W.llama_kv(dim=4096, heads=32, heads_kv=8, layers=layers, ff=14336, ctx=2048,
                                      vocab=["a"], rope=5e5, eps=1e-5), tensors)
        total = sum(len(t[3]) for t in tensors)
        names = [t[0] for t in tensors]
        del tensors
        with open(path, "rb") as f:  # page cache warm for both paths
            while f.read(1 << 26):
                pass
        g = gq.GGUF(path)
        info = {t["name"]: t for t in g.tensors()}
        outs = {nm: torch.empty(g.plan(nm, gq.LOAD_QUANT)["bytes"], dtype=torch.uint8, device=dev) for nm in names}

        def ours():
            for nm in names:
                o = outs[nm]
                g._check(gq.load().gq_gguf_load(g._h, nm.encode(), gq.LOAD_QUANT, gq._ptr(o), o.numel(),
                                                None, 0, None, 0), "gq_gguf_load")
            torch.cuda.synchronize()

        def reference_style():
            res = []
            with open(path, "rb") as f:
                for nm in names:
                    t = info[nm]
                    f.seek(t["offset"])
                    host = np.empty(t["size_bytes"], dtype=np.uint8)
                    f.readinto(host)
                    raw = torch.from_numpy(host).to(dev)
                    res.append(gq.repack(gq.FMT_Q4_K, raw, t["shape"][1], t["shape"][0]))
                    torch.cuda.synchronize()
            return res

        def ours_many():
            g.load_quant_many(names, [outs[nm] for nm in names])
            torch.cuda.synchronize()

        ours()  # staging buffers allocated here
        t0 = time.perf_counter()
        ours()
        t_ours = time.perf_counter() - t0
        t0 = time.perf_counter()
        ours_many()
        t_many = time.perf_counter() - t0
        t0 = time.perf_counter()
        ref = reference_style()
        t_ref = time.perf_counter() - t0
        same = all(torch.equal(outs[nm], r) for nm, r in zip(names, ref))
        del ref
        # the .greta T16 cache of the same tensors: a load is one upload, no repack
        gpath = os.path.join(d, "model.greta")
        t0 = time.perf_counter()
        gq.greta_write(g, gpath, gq.LOAD_QUANT)
        t_write = time.perf_counter() - t0
        g.close()
        with open(gpath, "rb") as f:
            while f.read(1 << 26):
                pass
        h = gq.Greta(gpath)
        gouts = {t["name"]: torch.empty(t["w_bytes"], dtype=torch.uint8, device=dev) for t in h.tensors()}

        def from_cache():
            for nm in names:
                o = gouts[nm]
                h._check(gq.load().gq_greta_load(h._h, nm.encode(), gq._ptr(o), o.numel(), None, 0, None, 0),
                         "gq_greta_load")
            torch.cuda.synchronize()

        from_cache()
        t0 = time.perf_counter()
        from_cache()
        t_cache = time.perf_counter() - t0
        same = same and all(torch.equal(outs[nm], gouts[nm]) for nm in names)
        h.close()
        return {"GBps": round(total / t_ours / 1e9, 2), "ms": round(t_ours * 1e3, 1), "bytes": total,
                "many_GBps": round(total / t_many / 1e9, 2),
                "reference_style_GBps": round(total / t_ref / 1e9, 2),
                "greta_cache_GBps": round(total / t_cache / 1e9, 2), "greta_write_s": round(t_write, 2),
                "same_bytes": same, "layers": layers, "format": "Q4_K",
                "note": "page-cache-warm files; H2D over PCIe"}
    finally:
        shutil.rmtree(d, ignore_errors=True)


def host_cores():
    """Cores this run may use, as `nproc` reports them (it honours
    OMP_NUM_THREADS and the CPU affinity mask)."""
    import subprocess
    try:
        return max(1, int(subprocess.run(["nproc"], capture_output=True, text=True, check=True).stdout.strip()))
    except (OSError, ValueError, subprocess.CalledProcessError):
        return len(os.sched_getaffinity(0))


def _time_cpu_gemv(fmt, n, k, seed, threads, target_s):
    """Repeated oracle GEMVs (dequant + fp64-accumulated dot, OpenMP over
    rows) for ~target_s seconds: (seconds per GEMV, repetitions, elapsed)."""
    import oracle as O
    w = O.gen_weights(fmt, n, k, seed=seed)
    x = O.gen_x(1, k, seed=seed + 1000)
    O.gemv(fmt, w, x, n, k, threads=threads)  # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        O.gemv(fmt, w, x, n, k, threads=threads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= target_s:
            return el / reps, reps, el


def cpu_baseline(target_s=6.0):
    """The oracle (C restatement of the reference CPU semantics: block dequant
    as weight_loader.cpp:91-156 / 703-712 and the GGUF spec, then a dot with
    fp64 accumulation as CpuReference::gemm, cpu_reference.hpp:56-66) on the
    host cores.  The headline workload (Q4_0 14336 x 4096, batch 1) on all
    cores gives `value`; the CPU-path configuration (Q8_0 4096 x 4096, batch
    1, x seed 0) is timed on all cores and on one, and the headline workload
    on one core too.  About 4 x target_s seconds in all."""
    import oracle as O
    cores = host_cores()
    runs = {}
    for name, fmt, n, k, seed in (("q4_0_14336x4096_b1", O.Q4_0, 14336, 4096, 1002),
                                  ("q8_0_4096x4096_b1", O.Q8_0, 4096, 4096, 1001)):
        for threads in (cores, 1):
            per, reps, el = _time_cpu_gemv(fmt, n, k, seed, threads, target_s)
            byts = gemv_bytes(fmt, n, k, 1)
            runs[f"{name}_{threads}t"] = {"GBps": round(byts / per / 1e9, 3), "ms_per_gemv": round(per * 1e3, 3),
                                          "threads": threads, "reps": reps, "seconds": round(el, 1)}
    head = runs[f"q4_0_14336x4096_b1_{cores}t"]
    return {"value": head["GBps"], "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"oracle gqo_gemv Q4_0 14336x4096 batch 1 on {cores} threads, {head['reps']} reps in "
                      f"{head['seconds']} s ({head['ms_per_gemv']} ms/GEMV); the other entries of 'runs' are the "
                      "Q8_0 4096x4096 batch-1 CPU-path configuration and single-thread runs",
            "runs": runs}


CALIB_PATH = os.path.join(ROOT, "gretacore-v3_amd", "lib", "libgqcalib.so")
_calib = None


def calib():
    """ctypes binding of lib/libgqcalib.so (gretacore-v3_amd/calib/gq_probe.h):
    calibration kernels, built beside the product library."""
    global _calib
    if _calib is None:
        import ctypes
        import torch  # noqa: F401  (torch's HIP runtime first, as gq.load())
        if not os.path.exists(CALIB_PATH):
            raise RuntimeError(f"{CALIB_PATH} not built (run __graft_entry__.build())")
        lib = ctypes.CDLL(CALIB_PATH)
        vp = ctypes.c_void_p
        lib.gq_probe_read.restype = ctypes.c_int
        lib.gq_probe_read.argtypes = [vp, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, vp, vp]
        lib.gq_probe_empty.restype = ctypes.c_int
        lib.gq_probe_empty.argtypes = [ctypes.c_int, ctypes.c_int, vp]
        lib.gq_probe_clock.restype = ctypes.c_int
        lib.gq_probe_clock.argtypes = [vp, ctypes.c_int, ctypes.c_int, vp]
        _calib = lib
    return _calib


def probe_read(src, wgs, waves, out):
    import torch
    s = torch.cuda.current_stream().cuda_stream
    rc = calib().gq_probe_read(src.data_ptr(), src.numel(), wgs, waves, out.data_ptr(), s)
    if rc != 0:
        raise RuntimeError(f"gq_probe_read: status {rc}")


def probe_empty(wgs, waves):
    import torch
    rc = calib().gq_probe_empty(wgs, waves, torch.cuda.current_stream().cuda_stream)
    if rc != 0:
        raise RuntimeError(f"gq_probe_empty: status {rc}")


def probe_clock_mhz(dev, iters=50000):
    """Effective shader clock (MHz) while every SIMD runs MFMA chains on
    changing operands (~20 ms): s_memtime ticks over s_memrealtime's 100 MHz
    ticks in one wave (the sysfs level is the DPM state, not the clock held
    under load)."""
    import torch
    out = torch.zeros(8, dtype=torch.int64, device=dev)
    rc = calib().gq_probe_clock(out.data_ptr(), 1024, iters, torch.cuda.current_stream().cuda_stream)
    if rc != 0:
        raise RuntimeError(f"gq_probe_clock: status {rc}")
    t0, t1, r0, r1 = (int(v) for v in out[:4].cpu())
    return round((t1 - t0) / max(1, r1 - r0) * 100.0, 1)


def bench_read_ceiling(dev, steps, warmup):
    """The read ceiling of the headline GEMV: a kernel of the GEMV's grid (its
    workgroups and waves, every wave issuing all its loads up front) that only
    streams the same bytes (the T16 Q4_0 14336 x 4096 tensor, rotated copies),
    and the same grid with no work (the fixed cost of a launch), in the same
    graph methodology as the GEMV."""
    import torch

    import gq
    import oracle as O
    n, k = 14336, 4096
    R, ks, _ = gq.gemv_plan(O.Q4_0, n, k, 1)
    wgs = -(-(-(-n // 16)) // R)
    nbytes = gq.packed_size(O.Q4_0, n, k)
    ncopies = max(8, -(-CACHE_DEFEAT_BYTES // nbytes))
    copies = [torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=dev) for _ in range(ncopies)]
    out = torch.empty(wgs * ks, dtype=torch.int32, device=dev)
    t_read = graph_steps(lambda i: probe_read(copies[i % ncopies], wgs, ks, out), steps, warmup)
    t_empty = graph_steps(lambda i: probe_empty(wgs, ks), steps, warmup)
    del copies
    return {"read_us": round(t_read * 1e6, 3), "read_GBps": round(nbytes / t_read / 1e9, 1),
            "read_pct_peak": round(100.0 * nbytes / t_read / 1e9 / HBM_PEAK_GBS, 2),
            "empty_us": round(t_empty * 1e6, 3), "bytes": nbytes, "grid": f"{wgs} workgroups x {ks} waves",
            "copies": ncopies}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--headline-only", action="store_true", help="only the headline GEMV (for profiling)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode-step", action="store_true")
    ap.add_argument("--no-load", action="store_true", help="skip the GGUF load-throughput extra")
    ap.add_argument("--only", default=None,
                    help="only the named GEMV config of the 'extra' field (e.g. q6_k_lm_head_128256x4096_b1), "
                         "after a 64 MiB copy for counter calibration; or one GEMM "
                         "(gemm_<fmt>_m<M>_<N>x<K>), read_ceiling (the headline's pure-read and empty kernels), "
                         "or decode_step_llama3_8b_q4k (for profiling)")
    ap.add_argument("--gemm-only", action="store_true",
                    help="only the Q4_0 M=2048 14336x4096 prefill GEMM, --steps times (for profiling)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (each GPU box has one GPU); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch

    import gq
    import oracle as O
    gq.load()
    dev = torch.device("cuda:0")
    steps, warmup = args.steps, args.warmup

    if args.gemm_only:
        r = bench_gemm(O.Q4_0, 2048, 14336, 4096, steps, warmup, dev)
        print(json.dumps({"gemm_q4_0_m2048_14336x4096": r}), flush=True)
        return
    gemv_cfgs = [("q8_0_4096x4096_b1", O.Q8_0, 4096, 4096, 1, 1001),
                 ("q8_0_lm_head_128256x4096_b1", O.Q8_0, 128256, 4096, 1, 1005),
                 ("q6_k_lm_head_128256x4096_b1", O.Q6_K, 128256, 4096, 1, 1006),
                 # the Q4 GEMV on a launch large enough that the launch ramp and
                 # tail stop mattering (the lm_head's shape): the rate it sustains
                 ("q4_0_128256x4096_b1", O.Q4_0, 128256, 4096, 1, 1007),
                 ("q4_k_128256x4096_b1", O.Q4_K, 128256, 4096, 1, 1008),
                 ("q4_0_4096x4096_b1", O.Q4_0, 4096, 4096, 1, 1002),
                 ("q4_0_4096x14336_b1", O.Q4_0, 4096, 14336, 1, 1002)]
    gemv_cfgs += [(f"q4_k_14336x4096_b{b}", O.Q4_K, 14336, 4096, b, 1003) for b in (1, 4, 8, 16)]
    if args.headline_only or args.only:
        # a plain copy of known size, so profiler byte counters can be
        # calibrated against the GEMV dispatches of the same run
        src = torch.empty(64 << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.bitwise_not(src, out=dst)  # reads 64 MiB, writes 64 MiB
        torch.cuda.synchronize()
        del src, dst
    if args.only and args.only.startswith("gemm_") and not args.only.startswith("gemm_q8_0_i8_"):
        # gemm_<fmt>_m<M>_<N>x<K>, e.g. gemm_q4_0_m64_4096x4096
        try:
            fname, rest = args.only[5:].rsplit("_m", 1)
            m_s, nk = rest.split("_", 1)
            n_s, k_s = nk.split("x")
            fmt = {"q4_0": O.Q4_0, "q8_0": O.Q8_0, "q4_k": O.Q4_K, "q6_k": O.Q6_K}[fname]
            m, n, k = int(m_s), int(n_s), int(k_s)
        except (ValueError, KeyError):
            print(f"--only: cannot parse {args.only} (gemm_<q4_0|q8_0|q4_k|q6_k>_m<M>_<N>x<K>)", file=sys.stderr)
            sys.exit(2)
        print(json.dumps({args.only: bench_gemm(fmt, m, n, k, steps, warmup, dev)}), flush=True)
        return
    if args.only and args.only.startswith("gemm_q8_0_i8_m"):
        # gemm_q8_0_i8_m<M>_<N>x<K>
        try:
            m_s, nk = args.only[len("gemm_q8_0_i8_m"):].split("_", 1)
            n_s, k_s = nk.split("x")
            m, n, k = int(m_s), int(n_s), int(k_s)
        except ValueError:
            print(f"--only: cannot parse {args.only} (gemm_q8_0_i8_m<M>_<N>x<K>)", file=sys.stderr)
            sys.exit(2)
        print(json.dumps({args.only: bench_gemm_q8_i8(m, n, k, steps, dev)}), flush=True)
        return
    if args.only == "read_ceiling":
        print(json.dumps({args.only: bench_read_ceiling(dev, steps, warmup)}), flush=True)
        return
    if args.only == "decode_step_llama3_8b_q4k":
        print(json.dumps({args.only: bench_decode_step(dev, steps, warmup)}), flush=True)
        return
    if args.only:
        cfg = [c for c in gemv_cfgs if c[0] == args.only]
        if not cfg:
            print(f"--only: unknown config {args.only}; one of {[c[0] for c in gemv_cfgs]}, "
                  "gemm_<fmt>_m<M>_<N>x<K>, read_ceiling or decode_step_llama3_8b_q4k", file=sys.stderr)
            sys.exit(2)
        name, fmt, n, k, b, seed = cfg[0]
        c = GemvCase(fmt, n, k, b, wseed=seed, xseed=seed + 1000, dev=dev)
        print(json.dumps({name: bench_gemv(c, steps, warmup)}), flush=True)
        return
    clock_mhz = {"before_headline": probe_clock_mhz(dev)}
    log("[bench] headline: Q4_0 GEMV 14336x4096 batch 1")
    head = GemvCase(O.Q4_0, 14336, 4096, 1, wseed=1002, xseed=2002, dev=dev)
    sysdir = gpu_sysfs_dir()
    with ClockSampler(sysdir) as clk_head:
        h = bench_gemv(head, steps, warmup)
    log(f"[bench] headline {h}")
    extra = {}
    log("[bench] read ceiling of the headline grid")
    rc = bench_read_ceiling(dev, steps, warmup)
    rc["gemv_over_read"] = round(h["step_us"] / rc["read_us"], 3)
    extra["read_ceiling_q4_0_14336x4096"] = rc
    if not args.headline_only:
        for name, fmt, n, k, b, seed in gemv_cfgs:
            log(f"[bench] {name}")
            c = GemvCase(fmt, n, k, b, wseed=seed, xseed=seed + 1000, dev=dev)
            extra[name] = bench_gemv(c, max(20, steps // 2), warmup)
            del c
            torch.cuda.empty_cache()
        log("[bench] fp16-weight lm_head (the reference's FP16 route)")
        extra["f16_lm_head_128256x4096_b1"] = bench_f16w(128256, 4096, 1, 20, 3, dev)
        torch.cuda.empty_cache()
        for fmt, fname in ((O.Q4_0, "q4_0"), (O.Q8_0, "q8_0"), (O.Q4_K, "q4_k")):
            for m in (64, 512, 2048):
                for n in (4096, 14336):
                    name = f"gemm_{fname}_m{m}_{n}x4096"
                    log(f"[bench] {name}")
                    with ClockSampler(sysdir) as clk:
                        extra[name] = bench_gemm(fmt, m, n, 4096, steps, warmup, dev)
                    if m == 2048 and n == 14336:
                        extra[name]["clock_during"] = clk.summary()
                    torch.cuda.empty_cache()
        clock_mhz["after_gemms"] = probe_clock_mhz(dev)
        log("[bench] int8 route for Q8_0 (per-32 activation quantization + int8 MFMA)")
        extra["gemm_q8_0_i8_m2048_14336x4096"] = bench_gemm_q8_i8(2048, 14336, 4096, steps, dev)
        torch.cuda.empty_cache()
        for m in (1, 512):
            log(f"[bench] reference INT4/INT8 launchers m={m}")
            extra[f"compat_launchers_14336x4096_m{m}"] = bench_compat(dev, m)
            torch.cuda.empty_cache()
        if not args.no_decode_step:
            log("[bench] decode step (config 5)")
            extra["decode_step_llama3_8b_q4k"] = bench_decode_step(dev, steps, warmup)
        if not args.no_load:
            log("[bench] GGUF-native load")
            extra["load_quant_q4_k_llama3_8b_8layers"] = bench_load(dev)
    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline")
        cpu = cpu_baseline()
    R, ks, cpw = gq.gemv_plan(O.Q4_0, 14336, 4096, 1)
    line = {
        "metric": "Q4 decode GEMV HBM GB/s (% peak) @14336x4096; prefill quant-GEMM TFLOPS",
        "value": round(h["GBps"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(h["step_us"] / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded GGUF Q4_0 blocks, x ~ N(0,1))",
        "config": {"workload": "Q4_0 decode GEMV 14336x4096 batch 1 (BASELINE configs[1]); one step = one "
                               "gq_gemv call (a single kernel) on one of the rotated weight copies; K steps "
                               "replayed from one HIP graph",
                   "N": 14336, "K": 4096, "batch": 1, "weight_copies_rotated": h["copies"],
                   "arithmetic": "Q4_0 codes x two int8 limbs of the activations per 32-block on the int8 "
                                 "MFMA, int32 products scaled and summed in f32",
                   "alg_bytes_per_step": h["alg_bytes"],
                   "box": dict(box_state(), clock_during_headline=clk_head.summary(),
                               sclk_under_mfma_load_mhz=clock_mhz)},
        "pct_peak": round(h["pct_peak"], 2),
        "rel_l2_vs_oracle": h["rel_l2"],
        "roofline": {"bound": "hbm", "achieved": round(h["GBps"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(h["GBps"] / HBM_PEAK_GBS, 4),
                     "traffic": PROFILED_TRAFFIC.get(("q4_0", 14336, 4096, 1, R, ks)),
                     "kernel": f"k_gemv_q<Q4_0, NB=1, R={R}, KSPLIT={ks}>",
                     "kernel_us": round(h["step_us"], 3),
                     "timing": "HIP events around the replay of K back-to-back launches; includes dispatch gaps"},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
