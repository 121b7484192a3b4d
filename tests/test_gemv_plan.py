"""CPU checks of the GEMV launch plan: for every shape the kernel is launched
with, each wave's chunk range and every weight load it issues (including the
surplus loads that re-read a chunk to keep the load count static) stay inside
the repacked tensor, and no wave holds more chunks than its registers."""
import pytest

import gq

MAXC = {gq.FMT_Q4_0: 8, gq.FMT_Q8_0: 8, gq.FMT_Q4_K: 4, gq.FMT_Q4_K_GGML: 4}
CK = {gq.FMT_Q4_0: 128, gq.FMT_Q8_0: 128, gq.FMT_Q4_K: 256, gq.FMT_Q4_K_GGML: 256}
QB = {gq.FMT_Q4_0: 1024, gq.FMT_Q8_0: 2048, gq.FMT_Q4_K: 2048, gq.FMT_Q4_K_GGML: 2048}

SHAPES = [(1, 32), (100, 288), (17, 96), (33, 160), (1, 256), (100, 256), (1, 768), (17, 512), (256, 2048),
          (4096, 4096), (14336, 4096), (4096, 14336), (1024, 4096), (128256, 4096), (7, 256), (40, 512)]


def emulate(fmt, n, k, batch):
    """Replays the kernel's chunk/address arithmetic on the host."""
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


@pytest.mark.parametrize("fmt", [gq.FMT_Q4_0, gq.FMT_Q8_0, gq.FMT_Q4_K])
@pytest.mark.parametrize("batch", [1, 2, 3, 4, 5, 8, 9, 16])
def test_gemv_plan_in_bounds(fmt, batch):
    for n, k in SHAPES:
        if k % (256 if fmt == gq.FMT_Q4_K else 32):
            continue
        emulate(fmt, n, k, batch)


def test_plan_single_chunk_has_idle_wave():
    # K = 32: one chunk, two waves -> one wave owns no chunk and must not index
    # chunk -1 (the address that faulted before the clamp was fixed)
    R, ks, cpw = gq.gemv_plan(gq.FMT_Q4_0, 1, 32, 1)
    assert ks >= 2 and cpw == 1
    emulate(gq.FMT_Q4_0, 1, 32, 1)
