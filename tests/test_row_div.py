"""The gathered GEMMs read token order[r] // top_k through a multiply-high
division by an invariant divisor (csrc/gemm_v2.hip: row_div_magic on the
host, div_rows in the kernel; the round-down method of Granlund and
Montgomery, PLDI 1994, with a 33-bit multiplier). This checks the method's
constants and steps against exact integer division on the CPU: every x below
2^16, multiples of d and their neighbours up to 2^31, and random x below
2^31, for every divisor the layer can use (top_k 1..64) and a few larger.
The kernel itself is checked against token ids in the gathered GEMM tests."""
import random

import pytest

MASK = (1 << 32) - 1


def magic(d):
    if d <= 1:
        return 0, 0
    s = 0
    while (1 << s) < d:
        s += 1
    return ((1 << 32) * ((1 << s) - d)) // d + 1, s


def div_rows(x, m, s):
    t = (x * m) >> 32
    q = ((t + (((x - t) & MASK) >> 1)) & MASK) >> (s - 1 if s > 0 else 0)
    return x if s == 0 else q


@pytest.mark.parametrize("d", list(range(1, 65)) + [96, 127, 255, 511])
def test_row_division_is_exact(d):
    m, s = magic(d)
    assert 0 <= m <= MASK
    rng = random.Random(d)
    xs = list(range(1 << 16))
    xs += [v for q in range(0, (1 << 31) // d, max(1, (1 << 31) // d // 4096))
           for v in (q * d - 1, q * d, q * d + 1, q * d + d - 1) if 0 <= v < (1 << 31)]
    xs += [rng.randrange(1 << 31) for _ in range(20000)] + [(1 << 31) - 1]
    for x in xs:
        assert div_rows(x, m, s) == x // d, (d, x)
