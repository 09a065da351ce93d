"""Host-side integer math the kernels rely on, checked on the CPU.

* FastDiv (csrc/common.hpp: make_fastdiv / fdiv): q = (umulhi(n, mul) + n) >> shift
  must equal n // d for every divisor the paged kernel may see (block sizes)
  and every token index below 2^31.
* The prefill grid's XCD-aware remap (csrc/flash_fwd.hip) must be a bijection
  from workgroup ids onto (batch, kv head, query tile, group member).
"""

from __future__ import annotations

import itertools
import random


def make_fastdiv(d: int) -> tuple[int, int]:
    s = 0
    while (1 << s) < d:
        s += 1
    return (((1 << 32) * ((1 << s) - d)) // d + 1) & 0xFFFFFFFF, s


def fdiv(n: int, mul: int, s: int) -> int:
    return (((n * mul) >> 32) + n) >> s


def test_fastdiv_exact():
    rng = random.Random(0)
    for d in list(range(1, 300)) + [1023, 1024, 4096, 65535, 100000, 2**20 + 7]:
        mul, s = make_fastdiv(d)
        assert mul < 2**32
        for n in list(range(0, 3000)) + [rng.randrange(0, 2**31) for _ in range(500)] + [2**31 - 1]:
            assert fdiv(n, mul, s) == n // d, (d, n)


def _remap(N, n_mt, G, Hk, B):
    seen = set()
    for bid in range(N):
        xcd, slot = bid & 7, bid >> 3
        logical = xcd * (N >> 3) + min(xcd, N & 7) + slot
        assert 0 <= logical < N
        per = n_mt * G
        grp, rem = divmod(logical, per)
        mt, g = n_mt - 1 - rem // G, rem % G
        b, kvh = divmod(grp, Hk)
        assert 0 <= mt < n_mt and 0 <= g < G and 0 <= kvh < Hk and 0 <= b < B
        seen.add((b, kvh, mt, g))
    return len(seen) == N


def test_prefill_grid_remap_is_bijective():
    for B, Hk, G, n_mt in itertools.product([1, 2, 3, 4], [1, 2, 3, 8], [1, 2, 4, 7], [1, 2, 5, 16, 33]):
        assert _remap(n_mt * B * Hk * G, n_mt, G, Hk, B)
