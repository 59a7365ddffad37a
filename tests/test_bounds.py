"""Byte ranges read by the device decoders, restated on the host: every load of a half-span
(Half<F>::ld) and of a span (Span<F>::w) in eureka-engine_amd/csrc/moe_dev.h stays inside the row.

A device read past a row is a read past the buffer for the last row of the last expert, which faults
the GPU when the stack ends on a page boundary (the C1 stacks do: 213,909,504 bytes). The address
arithmetic below follows the decoders line by line; a change there must be mirrored here.
"""
import pytest

BLK = {0: (4, 1), 1: (34, 32), 3: (144, 256), 9: (176, 256), 4: (210, 256)}  # format: (bytes, cols)


def al4(p):
    return p - (p & 3)


def half_reads(fm, c0, jh):
    """[start, end) byte ranges of Half<fm>::ld(row, c0, jh), row at 0 (rows are 16-aligned)."""
    b, n = BLK[fm]
    if fm == 0:
        s = 4 * (c0 + 16 * jh)
        return [(s, s + 64)]
    B = (c0 // n) * b
    if fm == 1:
        return [(B, B + 2), (B + 2 + 16 * jh, B + 18 + 16 * jh)]
    j = (c0 % 256) // 32
    if fm == 3:
        return [(B, B + 16), (B + 16 + 32 * (j >> 1) + 16 * jh, B + 32 + 32 * (j >> 1) + 16 * jh)]
    if fm == 9:
        return [(B, B + 16), (B + 16 + 16 * jh, B + 32 + 16 * jh),
                (B + 48 + 32 * (j >> 1) + 16 * jh, B + 64 + 32 * (j >> 1) + 16 * jh)]
    r = c0 % 256
    nn, quad = r >> 7, (r & 127) >> 5
    pl = B + 64 * nn + 32 * (quad & 1) + 16 * jh
    ph = B + 128 + 32 * nn + 16 * jh
    sc = B + 192 + (r >> 4) + jh
    return [(pl, pl + 16), (ph, ph + 16), (sc, sc + 1), (B + 208, B + 210)]


def span_reads(fm, c0):
    """[start, end) byte ranges of Span<fm>::w(row, c0)."""
    b, n = BLK[fm]
    if fm == 0:
        return [(4 * c0, 4 * c0 + 128)]
    B = (c0 // n) * b
    if fm == 1:
        a = al4(B)
        return [(a, a + 36)]  # nine aligned dwords
    j = (c0 % 256) // 32
    if fm == 3:
        return [(B, B + 16), (B + 16 + 32 * (j >> 1), B + 48 + 32 * (j >> 1))]
    if fm == 9:
        return [(B, B + 48), (B + 48 + 32 * (j >> 1), B + 80 + 32 * (j >> 1))]
    r = c0 % 256
    nn, quad = r >> 7, (r & 127) >> 5
    pl, ph = B + 64 * nn + 32 * (quad & 1), B + 128 + 32 * nn
    return [(al4(pl), al4(pl) + 36), (al4(ph), al4(ph) + 36), (B + 192 + 8 * nn + 2 * quad, B + 194 + 8 * nn + 2 * quad),
            (B + 208, B + 210)]


@pytest.mark.parametrize("fm", [0, 1, 3, 4, 9])
@pytest.mark.parametrize("cols", [256, 512, 768, 1536, 2048, 4096])
def test_decoder_reads_stay_in_the_row(fm, cols):
    b, n = BLK[fm]
    row = cols // n * b
    for c in range(0, cols, 32):
        for lo, hi in span_reads(fm, c) + half_reads(fm, c, 0) + half_reads(fm, c, 1):
            assert 0 <= lo < hi <= row, (fm, cols, c, lo, hi, row)


def test_the_fixed_q8_0_over_read_is_caught():
    """The earlier half-span helper read a half dword past its 16 bytes when the address was 4-aligned:
    for Q8_0's second half of an odd block that is 2 bytes past the block, past the row for the last one."""
    def old_half_q8(c0, jh):
        B = (c0 // 32) * 34
        p = B + 2 + 16 * jh
        a = al4(p)
        return [(B, B + 2), (a, a + 18)]  # four dwords and the half dword after them
    cols = 2048
    row = cols // 32 * 34
    assert max(hi for c in range(0, cols, 32) for jh in (0, 1) for _, hi in old_half_q8(c, jh)) == row + 2


# k_group's slot chunks (csrc/moe_q8.hip): thread t of 256 scans [t per, t per + per) with per rounded up to
# a multiple of 4; with per <= 64 its ids come through 16 quads, whole 16-byte loads only when the quad lies
# inside [i0, i1), single words for a ragged last quad
@pytest.mark.parametrize("n", [0, 1, 3, 8, 512, 513, 5130, 16384, 16385, 40000])
def test_group_chunks_in_range(n):
    per = ((n + 255) // 256 + 3) & ~3
    assert per % 4 == 0
    covered = []
    for t in range(256):
        i0 = min(t * per, n)
        i1 = min(i0 + per, n)
        covered.extend(range(i0, i1))
        if per <= 64:
            for q in range(16):
                i = i0 + 4 * q
                if not (4 * q < per and i < i1):
                    continue
                if i + 4 <= i1:
                    assert i % 4 == 0 and i + 4 <= n       # an aligned whole quad inside the ids
                else:
                    assert all(j < n for j in range(i, i1))  # the ragged tail: words below i1 only
    assert covered == list(range(n))                      # every slot once, in slot order


# the q8 tier's int8 GEMM decoders (eureka-engine_amd/csrc/moe_gemm.hip): i8_codes<F>(row, b, h) and
# i8_q6_half(row, b, k, h), restated
def i8_reads(fm, b, h):
    if fm == 1:
        B = 34 * b
        p = B + 2 + 16 * h
        rng = [(B, B + 2)]
        if p % 4 == 0:
            return rng + [(p, p + 16)]
        return rng + [(p, p + 2), (p + 2, p + 14), (p + 14, p + 16)]
    j = b & 7
    if fm == 3:
        B = 144 * (b >> 3)
        q = B + 16 + 32 * (j >> 1) + 16 * h
        return [(B, B + 16), (q, q + 16)]
    if fm == 9:
        B = 176 * (b >> 3)
        q = B + 48 + 32 * (j >> 1) + 16 * h
        return [(B, B + 16), (B + 16 + 16 * h, B + 32 + 16 * h), (q, q + 16)]
    raise ValueError(fm)


def i8_q6_reads(b, k, h):
    B = 210 * (b >> 3)
    bb = b & 7
    n, quad = bb >> 2, bb & 3
    i0 = 16 * k + 8 * h
    pl, ph = B + 64 * n + 32 * (quad & 1) + i0, B + 128 + 32 * n + i0
    sc = B + 192 + 8 * n + 2 * quad + k
    return [(pl, pl + 8), (ph, ph + 8), (B + 208, B + 210), (sc, sc + 1)]


@pytest.mark.parametrize("fm,cols", [(1, 32), (1, 64), (1, 768), (1, 2048), (3, 256), (3, 2048), (9, 512)])
def test_int8_gemm_codes_stay_inside_the_row(fm, cols):
    b_, n = BLK[fm]
    rb = cols // n * b_
    for b in range(cols // 32):
        for h in (0, 1):
            for s, e in i8_reads(fm, b, h):
                assert 0 <= s <= e <= rb, (fm, cols, b, h, s, e, rb)


def test_five_dword_q8_0_window_would_read_past_the_row():
    """the control: five aligned dwords from the code span (the loads this decoder had) end 4 bytes past
    the last block of a 2048-column Q8_0 row, so the checks above can see that mistake"""
    rb, B = 2176, 34 * 63
    p = B + 2 + 16
    assert p % 4 == 0 and p - (p & 3) + 20 > rb


@pytest.mark.parametrize("cols", [256, 512, 2048])
def test_int8_gemm_q6_halves_stay_inside_the_row(cols):
    rb = cols // 256 * 210
    for b in range(cols // 32):
        for k in (0, 1):
            for h in (0, 1):
                for s, e in i8_q6_reads(b, k, h):
                    assert 0 <= s < e <= rb, (cols, b, k, h, s, e, rb)
