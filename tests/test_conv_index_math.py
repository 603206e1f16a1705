"""Host-side checks of the integer index math the conv kernels use on the GPU
(csrc/icpp_kernels.hpp): the launch-constant division and the per-lane filter-tap
mask, each restated here and compared with brute force.  No GPU needed."""

import random

import pytest


def make_fastdiv(d):
    """(m, p) as icpp_abi.hip's make_fastdiv: p = 31 + ceil(log2 d), m = floor(2^p / d) + 1."""
    l = 0
    while (1 << l) < d:
        l += 1
    p = 31 + l
    m = (1 << p) // d + 1
    assert m < (1 << 32)
    return m, p


def fdiv(n, mp):
    m, p = mp
    return ((n & 0xFFFFFFFF) * m) >> p      # 64-bit product, then the shift (fits: n < 2^31, m < 2^32)


def test_fastdiv_matches_floor_division():
    rng = random.Random(7)
    divisors = list(range(1, 600)) + [2 ** k + o for k in range(1, 31) for o in (-1, 0, 1)] + \
        [rng.randrange(1, 2 ** 31) for _ in range(300)]
    for d in divisors:
        mp = make_fastdiv(d)
        ns = [0, 1, d - 1, d, d + 1, 2 ** 31 - 1, 2 ** 31 - 2, (2 ** 31 - 1) // d * d, (2 ** 31 - 1) // d * d - 1]
        ns += [rng.randrange(0, 2 ** 31) for _ in range(200)] + [k * d + r for k in (1, 7, 1000) for r in (0, d - 1)]
        for n in ns:
            if 0 <= n < 2 ** 31:
                assert fdiv(n, mp) == n // d, (n, d)


def tap_mask_loop(ih0, iw0, H, W, KH, KW, D=1):
    mk = 0
    for kh in range(KH):
        for kw in range(KW):
            ih, iw = ih0 + kh * D, iw0 + kw * D
            if 0 <= ih < H and 0 <= iw < W:
                mk |= 1 << (kh * KW + kw)
    return mk


def tap_mask_closed(ih0, iw0, H, W, KH, KW):
    """The dilation-1 closed form of the per-tile-tap gather's setup (32-bit unsigned arithmetic)."""
    U = 0xFFFFFFFF
    tap_rows = 0
    for kh in range(KH):
        if kh * KW < 32:
            tap_rows |= 1 << (kh * KW)
    kh_lo, kh_hi = max(0, -ih0), min(KH - 1, H - 1 - ih0)
    kw_lo, kw_hi = max(0, -iw0), min(KW - 1, W - 1 - iw0)
    if not (kh_lo <= kh_hi and kw_lo <= kw_hi):
        return 0
    cols = (((2 << kw_hi) - 1) & U) & ~((1 << kw_lo) - 1) & U
    rows = (((2 << ((kh_hi + 1) * KW - 1)) - 1) & U) & ~((1 << (kh_lo * KW)) - 1) & U
    return (cols * (tap_rows & rows)) & U


@pytest.mark.parametrize("KH,KW", [(3, 3), (1, 1), (5, 5), (1, 7), (7, 1), (2, 2), (4, 8), (8, 4), (2, 16), (32, 1), (1, 32)])
def test_tap_mask_closed_form_matches_loop(KH, KW):
    for H in (1, 2, 3, 5, 7, 14):
        for W in (1, 2, 4, 7, 9):
            for ih0 in range(-KH - 1, H + 2):
                for iw0 in range(-KW - 1, W + 2):
                    assert tap_mask_closed(ih0, iw0, H, W, KH, KW) == tap_mask_loop(ih0, iw0, H, W, KH, KW), \
                        (ih0, iw0, H, W, KH, KW)
