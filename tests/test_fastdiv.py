"""The multiply-shift division the RoPE kernel uses to split its flat thread
index (Granlund and Montgomery 1994): for a divisor d >= 2 with l = ceil(log2 d)
and m = ceil(2^(31+l) / d), floor(x / d) = (x * m >> 32) >> (l - 1) for every
0 <= x < 2^31. The host builds (m, l - 1) once per launch (make_fastdiv in
mla.hip); this checks the identity against integer division on the divisors
the kernel meets (threads per row, sequence lengths, head counts) and on edge
values, and the GPU RoPE tests check the kernel that uses it."""
import numpy as np
import pytest


def make(d):
    if d <= 1:
        return 0, 0
    l = int(d - 1).bit_length()          # ceil(log2 d)
    return ((1 << (31 + l)) + d - 1) // d, l - 1


@pytest.mark.parametrize("d", [1, 2, 3, 4, 5, 7, 8, 12, 16, 17, 24, 63, 64, 100, 128, 192, 2047,
                               2048, 4095, 4096, 8192, 16384, 65535, 1 << 20, (1 << 30) + 3])
def test_multiply_shift_division(d):
    m, s = make(d)
    assert m < 1 << 32
    rng = np.random.default_rng(d)
    x = np.concatenate([np.arange(0, 5000, dtype=np.uint64),
                        rng.integers(0, 1 << 31, 200000, dtype=np.uint64),
                        np.array([(1 << 31) - 1, (1 << 31) - 2, d - 1, d, d + 1,
                                  (((1 << 31) - 1) // d) * d, (((1 << 31) - 1) // d) * d - 1],
                                 dtype=np.uint64)])
    x = x[x < (1 << 31)]
    q = x if m == 0 else ((x * np.uint64(m)) >> np.uint64(32)) >> np.uint64(s)
    np.testing.assert_array_equal(q, x // np.uint64(d))
