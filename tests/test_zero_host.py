"""llb_hip_zero's fill kernel (k_zero in eureka-engine_amd/csrc/moe_q8.hip) restated on the host: for every
start alignment and sizes around the 16-byte body, every byte of [p, p + n) is written exactly once and
nothing outside it; the body's uint4 stores are 16-byte aligned. A change to the kernel must be mirrored
here."""
import numpy as np
import pytest


def cover(a, n):
    b0 = ((a + 15) & ~15) - a
    head = min(b0, n)
    body = (n - head) // 16
    tail0 = head + 16 * body
    units = (n + 15) // 16
    blocks = max(1, min(4096, (units + 255) // 256))
    nthr = blocks * 256
    cov = np.zeros(n, np.int32)
    for i in range(body):
        assert (a + head + 16 * i) % 16 == 0
    cov[head:head + 16 * body] += 1
    for i0 in range(min(nthr, 16)):
        if i0 < head:
            cov[i0] += 1
        if i0 < n - tail0:
            cov[tail0 + i0] += 1
    return cov


@pytest.mark.parametrize("a", range(0, 32))
def test_zero_fill_covers_each_byte_once(a):
    for n in list(range(1, 70)) + [4095, 4096, 4097, 65536 + 3]:
        assert (cover(a, n) == 1).all(), (a, n)
