"""The many-token router GEMV's index arithmetic (k_tree_rows_mt and its launcher launch_tree_rows in
eureka-engine_amd/csrc/moe_exact.hip), restated on the host and run over every block, wave, thread and
token tile: every global read of x and of the weight rows stays inside its buffer, every LDS access
inside the dynamic LDS the launcher sets, every token of every row is written exactly once, and no
write lands past T. Shapes: the 2048-token prefill, config 5's 513 tokens over 512 experts plus the
shared gate row, the 64-token batches, a ragged 33-token batch and the 4096-column two-span rows.
A change to the kernel's addressing or to the launcher's grid must be mirrored here.
"""
import numpy as np
import pytest


def launch(nsp, T, rows, cus=256):
    """launch_tree_rows' choice for T >= 16, nsp <= 2: TT, dynamic LDS bytes, ntb, grid, rows a wave"""
    tt, rw = 4, (4 if nsp == 1 else 2)
    sm = tt * 64 * (32 * nsp + 4) * 4
    nt, slots = (T + tt - 1) // tt, 2 * cus
    if (rows + 4 * rw - 1) // (4 * rw) * nt < slots:   # short of one round of resident blocks: a row a wave
        rw = 1
    rb = (rows + 4 * rw - 1) // (4 * rw)
    ntb, best = 1, None
    for n in range(1, nt + 1):
        cost = (rb * ((nt + n - 1) // n) + slots - 1) // slots * (n + 2)
        if best is None or cost < best:
            ntb, best = n, cost
    return tt, sm, ntb, (rb, (nt + ntb - 1) // ntb), rw


def test_tree_mt_tiles_a_block():
    for T, rows in ((513, 513), (2048, 128), (64, 128), (2048, 257)):
        TT, _, ntb, (gx, gy), _ = launch(1, T, rows)
        assert gx * gy <= 512 or ntb == 1   # one round of resident blocks unless a tile a block
        assert gy * ntb * TT >= T


def check(nsp, cols, T, segrows, wfmt_bytes=4):
    NQ = 8 * nsp
    LS4 = (4 * NQ + 4) // 4
    nl4 = cols // 4
    rows = sum(segrows)
    TT, sm, ntb, (gx, gy), RW = launch(nsp, T, rows)
    assert sm <= 160 * 1024
    lds4 = sm // 16
    tid = np.arange(256)
    L = tid & 63
    written = [np.zeros((T, r), np.int32) for r in segrows]
    # x staging: thread tid, load jj reads x row t0 + i / (64 NQ), float4 i % (64 NQ)
    XJ = TT * 64 * NQ // 256
    assert XJ * 256 == TT * 64 * NQ
    i = tid[:, None] + 256 * np.arange(XJ)[None, :]
    tts, li = i // (64 * NQ), i % (64 * NQ)
    st = tts * 64 * LS4 + (li // NQ) * LS4 + li % NQ
    assert st.min() >= 0 and st.max() < lds4
    rd = np.arange(TT)[:, None, None] * 64 * LS4 + L[None, :, None] * LS4 + np.arange(NQ)[None, None, :]
    assert rd.max() < lds4
    for by in range(gy):
        tb = by * TT * ntb
        for j in range(ntb):
            t0 = tb + j * TT
            if t0 >= T:
                break
            t = t0 + tts
            live = (t < T) & (li < nl4)
            assert (li[live] * 4 + 4 <= cols).all() and (t[live] < T).all()
        for bx in range(gx):
            for w in range(4):
                for k in range(RW):
                    r, s = bx * 4 * RW + RW * w + k, 0
                    while s < len(segrows) and r >= segrows[s]:
                        r -= segrows[s]
                        s += 1
                    if s >= len(segrows):
                        continue
                    assert r < segrows[s]
                    c0 = 32 * nsp * L
                    # weight bytes a lane reads: columns [c0, c0 + 32 nsp) of row r, for live lanes
                    lv = c0 < cols
                    assert ((c0[lv] + 32 * nsp) <= cols).all()
                    for j in range(ntb):
                        t0 = tb + j * TT
                        if t0 >= T:
                            break
                        for tt in range(TT):
                            if t0 + tt >= T:
                                break
                            written[s][t0 + tt, r] += 1
    for wr in written:
        assert (wr == 1).all()
    return ntb, gy


@pytest.mark.parametrize("nsp,cols,T,segrows", [
    (1, 2048, 2048, [128]),             # prefill router, 2048 tokens
    (1, 2048, 513, [512, 1]),           # config 5: 512 experts + the shared gate row
    (1, 2048, 64, [128]),               # 64-token batches (a row a wave)
    (1, 2048, 64, [256, 1]),
    (1, 1536, 33, [1000]),              # ragged: 33 tokens, 1000 rows, 1536 columns (dead lanes)
    (1, 2048, 16, [7, 1]),              # fewest tokens on this path, rows not a multiple of 8
    (2, 4096, 20, [40, 1]),             # two spans a lane
    (2, 4096, 1000, [64, 1]),
])
def test_tree_mt_indices(nsp, cols, T, segrows):
    check(nsp, cols, T, segrows)


def test_tree_mt_grid_covers_tokens():
    for T in (16, 17, 63, 64, 513, 2047, 2048, 4096):
        for rows in (1, 8, 129, 513, 1024):
            for nsp in (1, 2):
                TT, _, ntb, (gx, gy), RW = launch(nsp, T, rows, cus=(256, 80, 304)[(T + rows) % 3])
                assert gx * 4 * RW >= rows
                assert gy * ntb * TT >= T and (gy - 1) * ntb * TT < T


def test_tree_mt_rows_a_wave():
    assert launch(1, 64, 128)[4] == 1 and launch(1, 2048, 128)[4] == 4 and launch(1, 513, 513)[4] == 4
    assert launch(2, 20, 41)[4] == 1 and launch(2, 1000, 65)[4] == 2
