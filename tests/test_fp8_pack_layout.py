"""The packed fp8 weight layout of icpp_fp8_pack_b / icpp_fp8_gemm_packed, checked on the CPU.

`pack_ref` is the layout as one tensor permutation (the GPU tests compare the pack
kernel's bytes with it).  It is pinned here against the header's byte formula by
brute force over every byte, and the decode kernel's lane arithmetic is replayed
in numpy -- operand lane l of the 16x16x128 MFMA holding row / column l % 16 and K
slice 32 (l / 16) .. +32, result lane l holding m = 16 j + l % 16 (row tile j) and
n = 4 (l / 16) + e --
to show that fragments read that way from the packed B and from row-major A
reproduce A @ B exactly.  A planted mistake (the lane groups of B taken in the
wrong order) must break that equality.  No GPU needed.
"""

import numpy as np
import pytest
import torch


def pack_ref(b: torch.Tensor) -> torch.Tensor:
    """B [K, N] (any 1-byte dtype) -> the packed K * N bytes: index (nb, s, lane group g,
    lane row r, t) <- B[128 s + 32 g + t][16 nb + r]."""
    K, N = b.shape
    u = b.view(torch.uint8) if b.dtype != torch.uint8 else b
    return u.reshape(K // 128, 4, 32, N // 16, 16).permute(3, 0, 1, 4, 2).contiguous().reshape(-1)


@pytest.mark.parametrize("K,N", [(128, 16), (256, 48), (384, 32)])
def test_pack_ref_matches_the_byte_formula(K, N):
    g = torch.Generator().manual_seed(K + N)
    b = torch.randint(0, 256, (K, N), generator=g, dtype=torch.uint8)
    p = pack_ref(b).numpy()
    bn = b.numpy()
    S = K // 128
    for q in range(K * N):
        t, lane, blk = q % 32, (q // 32) % 64, q // 2048
        s, nb = blk % S, blk // S
        assert p[q] == bn[128 * s + 32 * (lane // 16) + t, 16 * nb + lane % 16], q


def decode_emulated(a: np.ndarray, bp: np.ndarray, M: int, N: int, K: int, b_group_order=(0, 1, 2, 3)) -> np.ndarray:
    """out[m][n] as the decode kernel forms it: per column block and K step, lane l's B
    fragment is bytes [32 l, 32 l + 32) of the step's 2 KiB, its A fragment row l % 16 at
    K offset 128 s + 32 (l / 16); the MFMA sums, over the 4 lane groups and 32 positions,
    B-fragment(lane 16 g + n % 16) x A-fragment(lane 16 g + m)."""
    S = K // 128
    MT = 1 if M <= 16 else 2           # row tiles of 16: rows 16 j + l % 16
    out = np.zeros((M, N), dtype=np.float64)
    a_pad = np.zeros((16 * MT, K), dtype=np.float64)
    a_pad[:M] = a
    for nb in range(N // 16):
        for s in range(S):
            step = bp[((nb * S + s) * 64) * 32:((nb * S + s) * 64 + 64) * 32].reshape(64, 32)
            for j in range(MT):
                for res_lane in range(64):
                    m, n0 = 16 * j + res_lane % 16, 4 * (res_lane // 16)
                    if m >= M:
                        continue
                    for e in range(4):
                        n = n0 + e
                        acc = 0.0
                        for g in range(4):
                            bfrag = step[16 * b_group_order[g] + n]
                            afrag = a_pad[m, 128 * s + 32 * g: 128 * s + 32 * g + 32]
                            acc += float(np.dot(bfrag, afrag))
                        out[m, 16 * nb + n] += acc
    return out


@pytest.mark.parametrize("M,N,K", [(1, 16, 128), (5, 32, 256), (16, 48, 384), (17, 16, 128), (32, 32, 256)])
def test_lane_arithmetic_reproduces_the_product(M, N, K):
    g = torch.Generator().manual_seed(M * 1000 + N + K)
    a = torch.randint(-3, 4, (M, K), generator=g).double().numpy()
    b = torch.randint(0, 7, (K, N), generator=g, dtype=torch.uint8)
    bp = pack_ref(b).numpy().astype(np.float64)
    got = decode_emulated(a, bp, M, N, K)
    want = a @ b.numpy().astype(np.float64)
    assert np.array_equal(got, want)


def test_the_emulation_catches_swapped_lane_groups():
    g = torch.Generator().manual_seed(7)
    M, N, K = 4, 16, 128
    a = torch.randint(-3, 4, (M, K), generator=g).double().numpy()
    b = torch.randint(0, 7, (K, N), generator=g, dtype=torch.uint8)
    bp = pack_ref(b).numpy().astype(np.float64)
    got = decode_emulated(a, bp, M, N, K, b_group_order=(1, 0, 2, 3))
    assert not np.array_equal(got, a @ b.numpy().astype(np.float64))
