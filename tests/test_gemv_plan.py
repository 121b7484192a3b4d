"""CPU checks of the GEMV launch plans: for every shape the kernels are
launched with, each wave's chunk range and every weight and activation load it
issues (including the surplus loads that re-read a chunk to keep the load count
static) stay inside the tensors, and no wave holds more chunks than its
registers.  Covers the int8 kernel (batch 1..4, and every batch through the
split gq_gemv_prep / gq_gemv_prepped form) and the fp16 batch kernel
(batch >= 5)."""
import os

import pytest

import gq

MAXC = {gq.FMT_Q4_0: 8, gq.FMT_Q8_0: 8, gq.FMT_Q4_K: 4, gq.FMT_Q4_K_GGML: 4, gq.FMT_Q6_K: 4}
CK = {gq.FMT_Q4_0: 128, gq.FMT_Q8_0: 128, gq.FMT_Q4_K: 256, gq.FMT_Q4_K_GGML: 256, gq.FMT_Q6_K: 256}
QB = {gq.FMT_Q4_0: 1024, gq.FMT_Q8_0: 2048, gq.FMT_Q4_K: 2048, gq.FMT_Q4_K_GGML: 2048, gq.FMT_Q6_K: 3072}

SHAPES = [(1, 32), (100, 288), (17, 96), (33, 160), (1, 256), (100, 256), (1, 768), (17, 512), (256, 2048),
          (4096, 4096), (14336, 4096), (4096, 14336), (1024, 4096), (128256, 4096), (7, 256), (40, 512)]


SB = {gq.FMT_Q4_0: 128, gq.FMT_Q8_0: 128, gq.FMT_Q4_K: 256, gq.FMT_Q4_K_GGML: 256, gq.FMT_Q6_K: 288}
KWIN = 256  # k per activation staging window of the fp16 batch kernel


def emulate_h(fmt, n, k, batch):
    """Replays k_gemv_h's window, chunk and address arithmetic on the host:
    workgroup = TW row tiles x KS parts of K, weights prefetched two windows
    ahead (clamped to the part's last chunk), MR (8 up to batch 8, else 16)
    activation rows staged per window in runs of 8."""
    TW, KS, cpw = gq.gemv_plan(fmt, n, k, batch)
    mr = 8 if batch <= 8 else 16
    assert TW in (1, 2, 4) and KS in (1, 2, 4, 8) and TW * KS <= 16
    assert 2 * TW <= mr  # x runs spread evenly over the threads
    C = -(-k // CK[fmt])
    assert KS <= C
    tiles = -(-n // 16)
    wc = KWIN // CK[fmt]
    assert cpw == -(-C // KS)
    NI = -(-cpw // wc)
    wgs = -(-tiles // TW)
    WB = KWIN * 2 * mr  # LDS bytes per part and window
    assert 2 * KS * WB <= 160 * 1024
    for part in range(KS):
        c0, c1 = C * part // KS, C * (part + 1) // KS
        assert 0 <= c0 < c1 <= C
        for it in range(max(NI, 2)):  # windows loaded: 0, 1 and it + 2 < NI
            for j in range(wc):
                ci = min(c0 + it * wc + j, c1 - 1)
                for blk in (0, wgs - 1):
                    for tt in range(TW):
                        t = min(blk * TW + tt, tiles - 1)
                        chunk = t * C + ci
                        assert chunk * QB[fmt] + QB[fmt] <= tiles * C * QB[fmt]
                        assert chunk * SB[fmt] + SB[fmt] <= tiles * C * SB[fmt]
        for it in range(NI):
            for kr in range(32):
                kk = c0 * CK[fmt] + 8 * kr + it * KWIN
                if kk < min(c1 * CK[fmt], k):
                    assert kk + 8 <= k  # a run of 8 is read only when wholly inside
    for run in range(KS * mr * 32):  # x runs of a window and their LDS destinations
        kr, b, p = run & 31, (run >> 5) % mr, run // (32 * mr)
        o = 8 * kr
        m, g, j = o >> 6, (o & 63) >> 4, (o & 15) >> 3
        dst = p * WB + (((m * 2 + j) * 4 + g) * mr + b) * 16
        assert 0 <= dst and dst + 16 <= KS * WB


def h1_plan(fmt, n, k, batch):
    """The one-stage fp16 kernel's plan (k_gemv_h1), or None where gq_gemv
    uses the windowed kernel: 4-bit formats, 16 waves as TW tiles x 16 / TW
    parts, MR (8 up to batch 8, else 16) activation rows of all of K in LDS
    (64 / 128 KiB: 2 / 1 workgroups per CU), one round of workgroups, grids
    of up to 512 row tiles."""
    if fmt not in (gq.FMT_Q4_0, gq.FMT_Q4_K):
        return None
    C = -(-k // CK[fmt])
    tiles = -(-n // 16)
    mr = 8 if batch <= 8 else 16
    slots = 256 * (2 if mr == 8 else 1)
    tw = 8
    while tw > 1 and -(-tiles // tw) < slots * 7 // 8:
        tw //= 2
    ks = 16 // tw
    if ks > C:
        return None
    nck = -(-C // ks)
    nckp = 1 if nck <= 1 else 2 if nck <= 2 else 4 if nck <= 4 else 8 if nck <= 8 else 16
    if nckp > (8 if fmt == gq.FMT_Q4_0 else 4) or ks * nckp * CK[fmt] * 2 * mr > (64 if mr == 8 else 128) * 1024:
        return None
    if tiles > 512:  # larger grids: the windowed kernel's 4-tile workgroups are faster
        return None
    if -(-tiles // tw) > slots:
        return None
    return tw, ks, nck


def emulate_h1(fmt, n, k, batch, plan):
    """Replays k_gemv_h1's chunk, activation-run and LDS arithmetic."""
    TW, KS, nck_max = plan
    C = -(-k // CK[fmt])
    tiles = -(-n // 16)
    wgs = -(-tiles // TW)
    mr = 8 if batch <= 8 else 16
    nckp = 1 if nck_max <= 1 else 2 if nck_max <= 2 else 4 if nck_max <= 4 else 8
    PK = nckp * CK[fmt]
    PB = PK * 2 * mr
    assert KS * PB <= 128 * 1024
    for part in range(KS):
        c0, c1 = C * part // KS, C * (part + 1) // KS
        assert 0 <= c0 < c1 <= C and c1 - c0 <= nckp
        for i in range(nckp):
            ci = min(c0 + i, c1 - 1)
            for blk in (0, wgs - 1):
                for tt in range(TW):
                    t = min(blk * TW + tt, tiles - 1)
                    assert (t * C + ci + 1) * QB[fmt] <= tiles * C * QB[fmt]
                    assert (t * C + ci + 1) * SB[fmt] <= tiles * C * SB[fmt]
    runs = KS * mr * (PK // 8)
    for run in range(runs):
        kr, b, p = run % (PK // 8), (run // (PK // 8)) % mr, run // (mr * (PK // 8))
        pc0, pc1 = C * p // KS, C * (p + 1) // KS
        kk = pc0 * CK[fmt] + 8 * kr
        if b < batch and kk < pc1 * CK[fmt] and kk < k:
            assert kk + 8 <= k
        o = 8 * kr
        ms, g, j = o >> 6, (o & 63) >> 4, (o & 15) >> 3
        dst = p * PB + (((ms * 2 + j) * 4 + g) * mr + b) * 16
        assert 0 <= dst and dst + 16 <= KS * PB
    # A reads: lane (g, r) at step ms, half j reads row r & (mr - 1)
    for part in range(KS):
        for ms in range(PK // 64):
            for j in range(2):
                for g in range(4):
                    for r in range(16):
                        off = part * PB + (g * mr + (r & (mr - 1))) * 16 + (ms * 2 + j) * 4 * mr * 16
                        assert off + 16 <= KS * PB


def emulate(fmt, n, k, batch):
    """Replays the int8 kernel's chunk/address arithmetic on the host."""
    R, ks, cpw = gq.gemv_plan(fmt, n, k, batch)
    C = -(-k // CK[fmt])
    tiles = -(-n // 16)
    nck_max = MAXC[fmt] // R
    assert cpw <= nck_max, (fmt, n, k, batch, R, ks, cpw)
    qs_plane = tiles * C * QB[fmt]
    wgs = -(-tiles // R)
    for wave in range(ks):
        c0, c1 = C * wave // ks, C * (wave + 1) // ks
        nck = c1 - c0
        assert 0 <= nck <= nck_max and 0 <= c0 < C and c1 <= C
        for blk in (0, wgs - 1):
            for rt in range(R):
                t = min(blk * R + rt, tiles - 1)
                for i in range(nck_max):
                    ii = i if i < nck else (nck - 1 if nck > 0 else 0)
                    chunk = t * C + c0 + ii
                    assert 0 <= chunk < tiles * C
                    assert chunk * QB[fmt] + QB[fmt] <= qs_plane


SHAPES_H = SHAPES + [(14336, 14336), (4096, 28672), (16, 65536)]


@pytest.mark.parametrize("fmt", [gq.FMT_Q4_0, gq.FMT_Q8_0, gq.FMT_Q4_K, gq.FMT_Q6_K])
@pytest.mark.parametrize("batch", [1, 2, 3, 4, 5, 8, 9, 16])
def test_gemv_plan_in_bounds(fmt, batch, monkeypatch):
    for n, k in SHAPES_H:
        if k % (32 if fmt in (gq.FMT_Q4_0, gq.FMT_Q8_0) else 256):
            continue
        # the int8 kernel holds up to 16 waves x MAXC chunks per row tile (K <=
        # 16384); Q6_K uses it at batch 1..2; the fp16 kernel takes the rest
        int8_fits = -(-k // CK[fmt]) <= 16 * MAXC[fmt]
        if batch >= 5 or (fmt == gq.FMT_Q6_K and batch > 2) or not int8_fits:
            p1 = h1_plan(fmt, n, k, batch)
            if p1 is not None:
                assert gq.gemv_plan(fmt, n, k, batch) == p1
                emulate_h1(fmt, n, k, batch, p1)
            else:
                emulate_h(fmt, n, k, batch)
        elif fmt == gq.FMT_Q6_K:
            emulate(fmt, n, k, batch)
    if fmt == gq.FMT_Q6_K:
        return
    # the int8 kernel at every batch (the split prep / prepped form uses it);
    # up to batch 4 gq_gemv stages the activation limbs in LDS, and where that
    # staging would exceed the 160 KiB of a workgroup even at a smaller K split
    # the fp16 kernel takes the shape instead (Q4_K 4096 x 16384 at batch 4)
    monkeypatch.setenv("GQ_GEMV_H_MIN", "17")
    for n, k in SHAPES:
        if k % (256 if fmt == gq.FMT_Q4_K else 32):
            continue
        if batch <= 4 and (staging_lds(fmt, n, k, batch) > 160 * 1024 or q8_spills(fmt, n, k, batch)):
            assert gq.gemv_plan(fmt, n, k, batch) != int8_plan(fmt, n, k, batch)
            emulate_h(fmt, n, k, batch)
            continue
        if batch <= 4:
            assert gq.gemv_plan(fmt, n, k, batch) == int8_plan(fmt, n, k, batch)
        emulate(fmt, n, k, batch)


def staging_lds(fmt, n, k, batch, ks=None, R=None):
    """LDS bytes of the int8 kernel at batch <= 4: the in-kernel activation
    staging (per wave, two int8 limb rows per batch row of the wave's K
    slice, a zero row and a float4 per (batch row, 32-block)) plus the
    kernel's static arrays (the scale-run copies where scales load by run, the
    K-split reduction tiles, the norm sums)."""
    if ks is None or R is None:
        R, ks, _ = int8_plan(fmt, n, k, batch)
    C = -(-k // CK[fmt])
    lk = CK[fmt] * -(-C // ks)
    wave = (2 * batch * lk + lk + batch * (lk // 32) * 16 + 15) & ~15
    nbc = 1 if batch == 1 else 2 if batch == 2 else 4
    sdma = fmt == gq.FMT_Q8_0 or (ks == 16 and fmt in (gq.FMT_Q4_0, gq.FMT_Q4_K, gq.FMT_Q4_K_GGML))
    static = (ks * R * 1024 if sdma else 16) + ks * R * nbc * 64 + nbc * 4
    return ks * wave + static


def q8_spills(fmt, n, k, batch):
    """Q8_0 at batch 3..4 on 16 waves with more than MAXC / 2 chunks a wave
    would spill registers (16 waves leave 128 a wave): the fp16 kernel."""
    R, ks, cpw = int8_plan(fmt, n, k, batch)
    return fmt == gq.FMT_Q8_0 and 3 <= batch <= 4 and ks == 16 and cpw > MAXC[fmt] // 2


def int8_plan(fmt, n, k, batch):
    """The int8 kernel's plan: the batch-1 plan, its K split halved while its
    LDS (batch <= 4) exceeds 160 KiB and the halved split's chunks per wave
    still fit MAXC / R."""
    R, ks, cpw = gq.gemv_plan(fmt, n, k, 1)
    C = -(-k // CK[fmt])
    while (batch <= 4 and ks > 2 and staging_lds(fmt, n, k, batch, ks, R) > 160 * 1024
           and -(-C // (ks // 2)) <= MAXC[fmt] // R):
        ks //= 2
    return R, ks, -(-C // ks)


def test_int8_staging_lds_guard():
    """Q4_K 4096 x 14336: at batch 4 the 16 waves would need 176 KiB of
    staging (3.5 KiB slices padded to 1024 k: 2 x 4 x 1024 + 1024 + 4 x 32 x
    16 bytes each) besides 20 KiB of static arrays, and a smaller split would
    need 7 chunks per wave (the registers hold 4): the fp16 batch kernel takes
    it.  Batch 3 stages its three rows only (136 KiB + 20 KiB) and stays on the
    int8 kernel.  Q4_0 at K = 14336, batch 4: 154 KiB of staging at 16 waves
    plus the static 20 KiB exceed the LDS, 8 waves would hold 14 chunks (the
    registers hold 8): the fp16 kernel; batch 3 stays on the int8 kernel."""
    assert staging_lds(gq.FMT_Q4_K, 4096, 14336, 4, 16, 1) == 16 * 11264 + 16384 + 4096 + 16
    assert gq.gemv_plan(gq.FMT_Q4_K, 4096, 14336, 4) != int8_plan(gq.FMT_Q4_K, 4096, 14336, 4)
    assert gq.gemv_plan(gq.FMT_Q4_K, 4096, 14336, 3) == (1, 16, 4) == int8_plan(gq.FMT_Q4_K, 4096, 14336, 3)
    assert staging_lds(gq.FMT_Q4_K, 4096, 14336, 3) == 16 * 8704 + 16384 + 4096 + 16 <= 160 * 1024
    assert staging_lds(gq.FMT_Q4_0, 4096, 14336, 4, 16, 1) > 160 * 1024
    assert gq.gemv_plan(gq.FMT_Q4_0, 4096, 14336, 4) != int8_plan(gq.FMT_Q4_0, 4096, 14336, 4)
    assert gq.gemv_plan(gq.FMT_Q4_0, 4096, 14336, 3) == (1, 16, 7) == int8_plan(gq.FMT_Q4_0, 4096, 14336, 3)


def test_plan_single_chunk_has_idle_wave():
    # K = 32: one chunk, two waves -> one wave owns no chunk and must not index
    # chunk -1 (the address that faulted before the clamp was fixed)
    R, ks, cpw = gq.gemv_plan(gq.FMT_Q4_0, 1, 32, 1)
    assert ks >= 2 and cpw == 1
    emulate(gq.FMT_Q4_0, 1, 32, 1)


def _emulate_int8_segment(fmt, n, k, R, ks):
    C = -(-k // CK[fmt])
    tiles = -(-n // 16)
    nck_max = MAXC[fmt] // R
    assert -(-C // ks) <= nck_max
    wgs = -(-tiles // R)
    for wave in range(ks):
        c0, c1 = C * wave // ks, C * (wave + 1) // ks
        nck = c1 - c0
        assert 0 <= c0 < C and c1 <= C
        for blk in (0, wgs - 1):
            for rt in range(R):
                t = min(blk * R + rt, tiles - 1)
                for i in range(nck_max):
                    ii = i if i < nck else (nck - 1 if nck > 0 else 0)
                    chunk = t * C + c0 + ii
                    assert 0 <= chunk < tiles * C


@pytest.mark.parametrize("fmt", [gq.FMT_Q4_0, gq.FMT_Q8_0, gq.FMT_Q4_K])
@pytest.mark.parametrize("batch", [1, 2, 4])
def test_fused_plans_in_bounds(fmt, batch):
    for ns, k in [((4096, 1024, 1024), 4096), ((14336,), 4096), ((64, 48, 16, 512), 1024), ((16,), 256),
                  ((4096, 4096, 4096), 4096), ((1024,), 14336)]:
        if k % (256 if fmt == gq.FMT_Q4_K else 32):
            continue
        R, ks, cpw = gq.gemv_multi_plan(fmt, list(ns), k, batch)
        if R == 0:  # the activation staging of a fused launch does not fit: gq_gemv_multi's fallback
            assert (R, ks, cpw) == (0, 0, 0) and batch >= 3 and k > 8192
            continue
        assert ks in (2, 4, 8, 16) and R in (1, 2)
        for n in ns:
            _emulate_int8_segment(fmt, n, k, R, ks)
    for n, k in [(14336, 4096), (16, 256), (100, 512), (11008, 4096)]:
        if k % (256 if fmt == gq.FMT_Q4_K else 32):
            continue
        ks, cpw = gq.gemv_swiglu_plan(fmt, n, k, batch)
        assert ks in (2, 4, 8, 16)
        _emulate_int8_segment(fmt, n, k, 2, ks)  # tile rt of workgroup i is tile i of gate / up
