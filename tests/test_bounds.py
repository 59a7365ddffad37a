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
