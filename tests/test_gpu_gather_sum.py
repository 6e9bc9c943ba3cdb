"""Scaled-table gather + sum (``lng_gather_sum_scaled``) against the oracle (GPU).

Rows are fixed by the oracle's integer restatement; the fp32 sums must match the fp64 oracle to
1e-5 norm-relative (and, for tables of small integers, exactly).  The full-size case is the
scaled-table configuration: 16 x 4096 tokens, 184 routes, orders (2, 3), tables grown 64x
(51,249,152 rows x 128 bf16 = 13.1 GB), checked on sampled tokens.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from lngram_hip import ops
from oracle import memory as om

pytestmark = pytest.mark.gpu


def _tables(R, orders, bits, sl, md, dtype, dev, gen, ints=False):
    out = []
    for n in orders:
        rows = R << (sl + bits * n)
        if ints:   # small integers: every fp32 partial sum is exact
            t = torch.randint(-8, 9, (rows, md), generator=gen).to(dtype)
        else:
            t = (torch.randn(rows, md, generator=gen) * 0.02).to(dtype)
        out.append(t.to(dev))
    return out


CASES = [  # B, T, R, orders, scale_log2, mem_dim, dtype
    (2, 37, 5, (2, 3), 3, 128, torch.bfloat16),
    (1, 9, 3, (1, 2, 3), 2, 32, torch.float32),
    (3, 1, 4, (2, 3), 1, 64, torch.bfloat16),      # T = 1: every row masked
    (1, 5, 7, (3,), 0, 16, torch.float32),         # one slot: the reference's rows
    (2, 11, 256, (2,), 0, 8, torch.bfloat16),      # 256 routes, 16-byte rows
]


@pytest.mark.parametrize("case", CASES)
def test_gather_sum_matches_oracle(dev, case):
    B, T, R, orders, sl, md, dt = case
    gen = torch.Generator().manual_seed(11)
    tabs = _tables(R, orders, 4, sl, md, dt, dev, gen)
    codes = torch.randint(0, 16, (B, T, R), generator=gen, dtype=torch.uint8)
    out = ops.gather_sum_scaled(tabs, codes.to(dev), orders, 4, sl, seed=1234)
    want = om.gather_sum_scaled([t.cpu() for t in tabs], codes.numpy(), orders, 4, sl, 1234)
    got = out.cpu().double().numpy()
    if T < max(orders):
        assert (got == 0).all()
    else:
        assert om.rel_err(torch.from_numpy(got), torch.from_numpy(want)) < 1e-5


def test_gather_sum_exact_on_integer_tables(dev):
    gen = torch.Generator().manual_seed(3)
    B, T, R, orders, sl = 2, 50, 9, (2, 3), 4
    tabs = _tables(R, orders, 4, sl, 128, torch.bfloat16, dev, gen, ints=True)
    codes = torch.randint(0, 256, (B, T, R), generator=gen, dtype=torch.uint8)   # high bits ignored
    got = ops.gather_sum_scaled(tabs, codes.to(dev), orders, 4, sl, seed=7).cpu().double().numpy()
    want = om.gather_sum_scaled([t.cpu() for t in tabs], codes.numpy(), orders, 4, sl, 7)
    assert (got == want).all()


def test_gather_sum_rejects_bad_shapes(dev):
    codes = torch.zeros(1, 4, 3, dtype=torch.uint8, device=dev)
    t2 = torch.zeros(3 * 256, 128, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        ops.gather_sum_scaled([t2], codes, (2,), 4, 1, 0)          # table not grown 2x
    t_bad = torch.zeros(3 * 256, 24, dtype=torch.bfloat16, device=dev)
    with pytest.raises(RuntimeError):
        ops.gather_sum_scaled([t_bad], codes, (2,), 4, 0, 0)       # 48-byte rows


def test_scaled_table_full_size_sampled(dev):
    """16 x 4096 tokens, R184, orders (2,3), 64 slots per route: 13.1 GB bf16 table."""
    B, T, R, orders, sl, md = 16, 4096, 184, (2, 3), 6, 128
    print(f"[scaled full size] B{B} T{T} R{R} S{1 << sl}", flush=True)
    n2, n3 = R << (sl + 8), R << (sl + 12)
    table = torch.empty(n2 + n3, md, dtype=torch.bfloat16, device=dev)
    g = torch.Generator(device=dev).manual_seed(0)
    for s0 in range(0, n2 + n3, 1 << 22):
        blk = table[s0:s0 + (1 << 22)]
        blk.copy_(torch.randn(blk.shape, generator=g, device=dev, dtype=torch.float32).mul_(0.02))
    tabs = [table[:n2], table[n2:]]
    codes = torch.randint(0, 16, (B, T, R), generator=torch.Generator().manual_seed(5), dtype=torch.uint8)
    out = ops.gather_sum_scaled(tabs, codes.to(dev), orders, 4, sl, seed=2024)
    torch.cuda.synchronize()
    rng = np.random.default_rng(0)
    pos = np.concatenate([[0, 1, 2, T - 1, T, T + 1, B * T - 1], rng.integers(0, B * T, 57)])
    want = om.gather_sum_scaled(tabs, codes.numpy(), orders, 4, sl, 2024, positions=pos)
    got = out.view(B * T, md)[torch.from_numpy(pos).to(dev)].cpu().double().numpy()
    assert om.rel_err(torch.from_numpy(got), torch.from_numpy(want)) < 1e-5
    assert (got[0] == 0).all() and np.abs(got[1]).sum() > 0
    del table, tabs, out
    torch.cuda.empty_cache()
