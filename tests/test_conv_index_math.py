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


def _halo_tile(Nb, H, W, BM, MF, row0, wave_rows):
    """The A_HALO tile of 64 channels starting at output row row0, as the kernel lays it out
    (icpp_kernels.hpp setup_halo / issue_halo / load_frags): the LDS image the loader writes
    -- {slot: (n, h, w, logical chunk) or None for zeros} -- and, per (output pixel, tap,
    lane K chunk), the LDS slot the fragment read takes."""
    M = Nb * H * W
    g0 = row0 // W
    rows = (min(row0 + BM, M) - 1) // W - g0 + 3
    zpix = rows * W
    swz = (lambda q: q & 7) if MF == 16 else (lambda q: (q >> 1) & 7)
    lds = {}
    for s in range((zpix + 1) * 8):                 # issue_halo
        q = s >> 3
        pix = (g0 - 1) * W + q
        chunk = (s & 7) ^ swz(q)
        ok = q < zpix and 0 <= pix < M
        lds[s] = (pix // (H * W), pix % (H * W) // W, pix % W, chunk) if ok else None
    reads = {}
    for r in range(wave_rows):                      # setup_halo + load_frags, one lane row each
        m = min(row0 + r, M - 1)
        g, ow = divmod(m, W)
        oh = g % H
        hq = (g - g0) * W + ow - 1
        rm = (oh > 0) | 2 | ((oh < H - 1) << 2)
        cm = (ow > 0) | 2 | ((ow < W - 1) << 2)
        vmask = (cm if rm & 1 else 0) | ((cm << 3) if rm & 2 else 0) | ((cm << 6) if rm & 4 else 0)
        for tap in range(9):
            kh, kw = divmod(tap, 3)
            q = hq + kh * W + kw if (vmask >> tap) & 1 else zpix
            for kgrp in range(4 if MF == 16 else 2):   # lane K chunk within a K-step
                for h_chunk in ((0, 4) if MF == 16 else (0, 2, 4, 6)):
                    pa = (q << 7) + ((kgrp ^ swz(q)) << 4)
                    off = pa ^ (h_chunk << 4)
                    reads[(r, tap, h_chunk + kgrp)] = (m, off // 16)
    return lds, reads


@pytest.mark.parametrize("geo", [(3, 9, 11, 256, 16), (2, 13, 5, 256, 16), (1, 56, 56, 256, 32), (4, 7, 7, 64, 16),
                                 (2, 6, 14, 224, 16)])
def test_halo_reads_fetch_the_tap_input_or_zero(geo):
    """Every (output pixel, tap, 16-byte K chunk) the fragment reads of an A_HALO tile take
    from LDS holds input pixel (n, oh + kh - 1, ow + kw - 1), channels 8 * chunk .. + 7, or
    zeros when that pixel lies outside the image -- checked against the definition of the
    3x3 stride-1 pad-1 conv for every tile of the shape (brute force over the loader's LDS
    image)."""
    Nb, H, W, BM, MF = geo
    M = Nb * H * W
    for row0 in range(0, M, BM):
        lds, reads = _halo_tile(Nb, H, W, BM, MF, row0, min(BM, M - row0))
        for (r, tap, chunk), (m, slot) in reads.items():
            n, rem = divmod(m, H * W)
            oh, ow = divmod(rem, W)
            kh, kw = divmod(tap, 3)
            ih, iw = oh + kh - 1, ow + kw - 1
            want = (n, ih, iw, chunk) if 0 <= ih < H and 0 <= iw < W else None
            assert lds[slot] == want, (geo, row0, r, tap, chunk)
