"""CPU models of the 16x16x32 GEMM kernel's address arithmetic
(``csrc/hmx_gemm_mi16.hpp``): what its direct-to-LDS loads fetch and where
they land, and what its fragment reads then hold.

* VNNI panels ``[N/P, Kp/2, P, 2]`` (``pack_b_vnni_t``; ``pack_b_blocked_vnni``
  is panels of 32, ``matmul.py:947-970`` of the reference) are re-laid as they
  land: each lane of a 1 KiB load picks a 16-byte piece (4 columns of one K
  pair). The model fills an LDS stage from tagged global data with the
  kernel's lane and load offsets, then reads every lane's fragments with the
  kernel's read offsets, and checks each value's (k, n), that each read
  instruction meets 64 distinct banks, that each load reads whole 128-byte
  rows, and that every byte read lies inside B.
* Ragged tiles (M or N not whole tiles): the clamped offsets keep every
  buffer load inside the operand's span (the scalar offset of a buffer load
  is not range-checked, so the kernel keeps rows and columns in the vector
  offset).

The GPU tests (``test_gpu_gemm.py``, ``test_gpu_packed.py``) check the same
layouts end to end, bit-equal to the plain kernel.
"""

from __future__ import annotations

import numpy as np
import pytest

LANES = np.arange(64)


def _vnni_lane_part(p: int, kpad: int) -> np.ndarray:
    f = (LANES >> 2) & 3
    lam = 16 * (LANES >> 4) + 4 * (LANES & 3)
    return f * 16 * p + (lam // p) * (kpad // 2) * 4 * p + (lam % p) * 4


def _vnni_load_part(p: int, kpad: int, n0: int, b: int) -> int:
    ks, i, col = b >> 4, (b >> 2) & 3, n0 + 64 * (b & 3)
    return (16 * ks + i) * 4 * p + (col // p) * (kpad // 2) * 4 * p + (col % p) * 4


@pytest.mark.parametrize("panel", [32, 64, 128, 256, 512, 768])
def test_vnni_stage_relayout(panel: int) -> None:
    kpad, k0 = 320, 128  # stage 2 of a 320-deep product
    tiles = [n0 for n0 in (0, 256, 512) if panel > 256 or n0 % panel == 0]
    n = max(tiles) + 256
    panels = -(-n // panel)
    # Tagged B: element (k, col) holds k * 100000 + col, VNNI-panel order.
    kk = np.arange(kpad)[:, None]
    cc = np.arange(panels * panel)[None, :]
    tags = kk * 100000 + cc  # [K, N]
    g = tags.reshape(kpad // 2, 2, panels, panel).transpose(2, 0, 3, 1).reshape(-1)
    b_bytes = g.size * 2
    lane_part = _vnni_lane_part(panel, kpad)
    for n0 in tiles:
        lds = np.full(16 * 1024, -1, dtype=np.int64)  # the 32 KiB B stage, bf16 elements
        for b in range(32):  # load b = wave * 4 + q of the 8 waves' 4 loads
            src = (k0 // 2) * 4 * panel + _vnni_load_part(panel, kpad, n0, b) + lane_part
            assert (src % 16 == 0).all() and src.min() >= 0 and (src + 16).max() <= b_bytes
            rows = np.unique(src // 128)
            assert len(rows) == 8 and all(((src // 128) == r).sum() == 8 for r in rows)
            dst = (b * 1024 + LANES * 16) // 2
            for e in range(8):
                lds[dst + e] = g[src // 2 + e]
        assert (lds >= 0).all()
        frow, fg = LANES & 15, LANES >> 4
        for wn in range(4):
            for j in range(4):
                base = (wn * 4 + j) * 256 + fg * 64 + frow * 4
                col = n0 + wn * 64 + 16 * j + frow
                for ks in range(2):
                    got = []
                    for i in range(4):
                        addr = base + ks * 16384 + i * 4096
                        banks = (addr // 4) % 64
                        assert len(np.unique(banks)) == 64
                        got += [lds[addr // 2], lds[addr // 2 + 1]]
                    want = [(k0 + 32 * ks + 8 * fg + e) * 100000 + col for e in range(8)]
                    np.testing.assert_array_equal(np.stack(got), np.stack(want))


def _kc_voff(ld: int, rows: np.ndarray, nrows: int, par: int) -> np.ndarray:
    rr, slot = LANES >> 3, LANES & 7
    return (np.minimum(rows, nrows - 1) * ld + (slot ^ ((rr >> 1) | (par << 2))) * 8) * 2


@pytest.mark.parametrize("m,n,k", [(4000, 4000, 4096), (3000, 11008, 4096), (1000, 4104, 256), (300, 200, 128)])
def test_ragged_loads_stay_inside_the_operands(m: int, n: int, k: int) -> None:
    # A [M, K] and K-contiguous B [N, K] (ld = K): eight waves, four 1 KiB
    # loads of 8 rows each; row-major B [K, N] (ld = N): rows 8 w .. + 7 in
    # pairs, columns clamped to the last 8-column chunk.
    for rows, ld, bm in ((m, k, 256), (n, k, 256)):
        span = ((rows - 1) * ld + k) * 2
        for t0 in range(0, -(-rows // bm) * bm, bm):
            for wave in range(8):
                for q in range(4):
                    r = t0 + wave * 32 + q * 8 + (LANES >> 3)
                    v = _kc_voff(ld, r, rows, q & 1)
                    for k0 in (0, k - 64):
                        assert v.min() + k0 * 2 >= 0 and (v + k0 * 2 + 16).max() <= span
    span = ((k - 1) * n + n) * 2
    last = ((n - 1) >> 3) << 3
    r, c = LANES >> 5, LANES & 31
    for n0 in range(0, -(-n // 256) * 256, 256):
        for wave in range(8):
            cw = c ^ (((wave * 8) >> 2) & 2)
            for qb in range(4):
                sw = ((r + 2 * (qb & 1)) & 3)
                chunk = cw ^ (((sw & 3) << 1) ^ ((sw & 3) << 2))
                col = np.minimum(n0 + chunk * 8, last)
                for k0 in (0, k - 64):
                    row = k0 + wave * 8 + 2 * qb + r
                    off = (row * n + col) * 2
                    assert off.min() >= 0 and (off + 16).max() <= span
