"""Oracle of the scaled-table gather + sum (CPU): the slot hash and the scaled rows.

Pins: MurmurHash3 fmix32 known answers (fmix32(0) = 0, fmix32(1) = 0x514e28b7) and its
inverse; with one slot per route the scaled rows are the reference's global rows (pinned by the
reference's address known answers in test_oracle_codes.py); every row lies in its route's block;
slots are uniform; the vectorised rows equal a per-entry loop over the definition.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import memory as om


def _inv_mix32(h: int) -> int:
    """Inverse of fmix32 (xorshift inverses and modular inverses of the two multipliers)."""
    M = 0xFFFFFFFF

    def unxorshift(x, s):
        y = x
        for _ in range(32 // s + 1):
            y = x ^ (y >> s)
        return y & M

    h = unxorshift(h, 16)
    h = (h * pow(0xC2B2AE35, -1, 1 << 32)) & M
    h = unxorshift(h, 13)
    h = (h * pow(0x85EBCA6B, -1, 1 << 32)) & M
    return unxorshift(h, 16)


def test_mix32_known_answers_and_bijection():
    assert int(om.mix32(0)) == 0
    assert int(om.mix32(1)) == 0x514E28B7
    xs = np.random.default_rng(0).integers(0, 1 << 32, 500, dtype=np.uint64)
    hs = om.mix32(xs)
    assert all(_inv_mix32(int(h)) == int(x) for h, x in zip(hs, xs))


def test_scale_one_is_reference_rows():
    c = np.random.default_rng(1).integers(0, 16, (3, 11, 7))
    for seed in (0, 5, 0xFFFFFFFF):
        assert (om.scaled_rows(c, (2, 3), 4, 0, seed) == om.route_rows(c, (2, 3), 4)).all()


def test_rows_in_route_blocks_and_uniform_slots():
    rng = np.random.default_rng(2)
    c = rng.integers(0, 256, (4, 300, 6))                  # codes above 2^bits are masked to bits
    S = 8
    rows = om.scaled_rows(c, (2, 3), 4, 3, 11)
    for oi, n in enumerate((2, 3)):
        r = rows[..., oi]
        assert (r[:, : n - 1] == -1).all() and (r[:, n - 1:] >= 0).all()
        blk = S << (4 * n)
        route = np.arange(6)[None, None, :]
        ok = r[:, n - 1:]
        assert ((ok >= route * blk) & (ok < (route + 1) * blk)).all()
        slot = (ok % blk) >> (4 * n)
        hist = np.bincount(slot.ravel(), minlength=S)
        exp = slot.size / S
        chi2 = ((hist - exp) ** 2 / exp).sum()
        assert chi2 < 30, chi2                               # 7 dof: p ~ 1e-4


def test_rows_match_per_entry_definition():
    rng = np.random.default_rng(3)
    b, t, r, orders, bits, sl, seed = 2, 6, 3, (1, 2, 3), 4, 2, 99
    c = rng.integers(0, 16, (b, t, r))
    got = om.scaled_rows(c, orders, bits, sl, seed)
    for bi in range(b):
        for ti in range(t):
            p = bi * t + ti
            for ri in range(r):
                for oi, n in enumerate(orders):
                    if ti < n - 1:
                        assert got[bi, ti, ri, oi] == -1
                        continue
                    addr = sum(int(c[bi, ti - n + 1 + k, ri]) << (bits * k) for k in range(n))
                    h = (p * 0x9E3779B1 + ri * len(orders) + oi) & 0xFFFFFFFF
                    slot = int(om.mix32(seed ^ int(om.mix32(h)))) & ((1 << sl) - 1)
                    assert got[bi, ti, ri, oi] == ((ri << sl) + slot) * (1 << (bits * n)) + addr


def test_gather_sum_of_constant_tables_counts_rows():
    c = np.random.default_rng(4).integers(0, 16, (2, 5, 3))
    tabs = [torch.ones(3 * 2 * 256, 8), torch.ones(3 * 2 * 4096, 8)]
    out = om.gather_sum_scaled(tabs, c, (2, 3), 4, 1, 0)
    want = np.array([0, 3, 6, 6, 6], float)                # t=0: none, t=1: 2-grams, t>=2: both
    assert (out[..., 0] == want[None]).all()


def test_torch_gather_sum_agrees_with_the_fp64_restatement():
    g = torch.Generator().manual_seed(5)
    c = np.random.default_rng(6).integers(0, 16, (2, 9, 5))
    tabs = [torch.randn(5 * 4 * 256, 16, generator=g).to(torch.bfloat16),
            torch.randn(5 * 4 * 4096, 16, generator=g).to(torch.bfloat16)]
    want = om.gather_sum_scaled(tabs, c, (2, 3), 4, 2, 11)
    got = om.gather_sum_rows_torch(tabs, om.scaled_rows(c, (2, 3), 4, 2, 11))
    assert got.dtype == torch.float32 and got.shape == want.shape
    assert om.rel_err(got.double(), torch.from_numpy(want)) < 1e-6   # bf16 rows are exact in fp32
    assert (got[:, 0] == 0).all()                                     # t = 0 reads no row
