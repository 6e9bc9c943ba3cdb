"""The oracle's lookup-surrogate gradient (``oracle.memory.surrogate_grad``; the backward of
``_LngramSurrogate``, ``lngram_v2.py:328-464``), pinned three ways on the CPU:

- the reference's own gradients (``tests/golden/surrogate.npz``, written by ``make_golden.py``
  from ``_LngramSurrogate.apply(...).backward``), approximate and exact, fp32 and bf16 tables,
  orders 2 and 3, 2- and 4-bit codes, a route offset and an invalid position;
- the exact mode is the derivative of an expected dot product, so it equals central finite
  differences of ``surrogate_expected_dot`` (brute force in fp64);
- for a table that is linear in the address bits, the counterfactual difference of every bit is
  that bit's weight vector, which gives the approximate mode in closed form; the exact mode then
  agrees with it (the bits are independent).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import memory as om

GOLD = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLD))
import recipe  # noqa: E402


def case_inputs(case):
    """Tensors of one fixture case, built as make_golden.py built them."""
    name, order, bits, R, rs, B, T, D, dt_name, temp, scale, exact = case
    dt = torch.bfloat16 if dt_name == "bf16" else torch.float32
    x = recipe.surrogate_inputs(case)
    table = torch.from_numpy(x["table"]).to(dt)
    codes = x["codes"]
    valid = om.valid_mask(order, B, T, valid_tokens=x["valid_tokens"])
    rows = om.route_rows(codes, [order], bits, 0, R, valid_tokens=x["valid_tokens"])[..., 0]
    rows = np.where(rows >= 0, rows + rs * (1 << (bits * order)), -1)
    hard = table[torch.from_numpy(rows).clamp_min(0)] * torch.from_numpy(rows >= 0)[..., None].to(dt)
    return dict(table=table, codes=codes, valid=valid, hard=hard, q=torch.from_numpy(x["q"]),
                grad=torch.from_numpy(x["grad"]).to(dt))


def _gold() -> dict:
    with np.load(GOLD / "surrogate.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("case", recipe.SURROGATE_CASES, ids=[c[0] for c in recipe.SURROGATE_CASES])
def test_surrogate_grad_matches_reference(case):
    name, order, bits, R, rs, B, T, D, dt_name, temp, scale, exact = case
    x = case_inputs(case)
    g = _gold()
    got = om.surrogate_grad(x["grad"], x["hard"], x["q"], x["codes"], x["table"], x["valid"], order, bits, rs,
                            temp, scale, exact)
    want = torch.from_numpy(g[f"{name}_grad_q"]).double()
    assert want.abs().max() > 0
    assert om.rel_err(got, want) < 1e-5
    # the memory gradient passes through unchanged
    gm = g[f"{name}_grad_mem"]
    gm = torch.from_numpy(gm.view(np.int16)).view(torch.bfloat16) if dt_name == "bf16" else torch.from_numpy(gm)
    assert torch.equal(gm, x["grad"])


@pytest.mark.parametrize("order,bits", [(2, 2), (3, 1), (2, 3)])
def test_exact_mode_is_the_derivative_of_the_expected_dot(order, bits):
    gen = torch.Generator().manual_seed(order * 10 + bits)
    B, T, R, D, rs = 1, 5, 2, 6, 1
    A = 1 << bits
    table = torch.randn((rs + R) * A ** order, D, generator=gen, dtype=torch.float64)
    codes = torch.randint(0, A, (B, T, R), generator=gen).numpy()
    q = torch.randn(B, T, R, bits, generator=gen, dtype=torch.float64)
    grad = torch.randn(B, T, R, D, generator=gen, dtype=torch.float64)
    vt = np.ones((B, T), bool)
    vt[0, T - 1] = False
    valid = om.valid_mask(order, B, T, valid_tokens=vt)
    temp, scale = 0.8, 1.7
    hard = torch.zeros(B, T, R, D, dtype=torch.float64)        # the exact mode does not read it
    got = om.surrogate_grad(grad, hard, q, codes, table, valid, order, bits, rs, temp, scale, True)
    h = 1e-6
    fd = torch.zeros_like(q)
    for i in np.ndindex(*q.shape):
        qp, qm = q.clone(), q.clone()
        qp[i] += h
        qm[i] -= h
        fp = om.surrogate_expected_dot(qp, codes, table, grad, valid, order, bits, rs, temp, scale)
        fm = om.surrogate_expected_dot(qm, codes, table, grad, valid, order, bits, rs, temp, scale)
        fd[i] = (fp - fm) / (2 * h)
    assert fd.abs().max() > 0
    assert om.rel_err(got, fd) < 1e-7


@pytest.mark.parametrize("order,bits", [(2, 4), (3, 4), (3, 2)])
def test_linear_table_closed_form(order, bits):
    """table[(rs + r) * A^n + addr] = w0[r] + sum_j bit_j(addr) v[r, j]: flipping bit j moves the
    row by +-v[r, j], so position t's score for bit k is the sum over its windows of v[r, e*bits+k] . g."""
    gen = torch.Generator().manual_seed(7 * order + bits)
    B, T, R, D, rs = 2, 8, 3, 5, 2
    A = 1 << bits
    nbit = order * bits
    w0 = torch.randn(rs + R, D, generator=gen, dtype=torch.float64)
    v = torch.randn(rs + R, nbit, D, generator=gen, dtype=torch.float64)
    addr = torch.arange(A ** order)
    addr_bits = ((addr[:, None] >> torch.arange(nbit)) & 1).double()            # [A^n, nbit]
    table = (w0[:, None, :] + torch.einsum("aj,rjd->rad", addr_bits, v)).reshape(-1, D)
    codes = torch.randint(0, A, (B, T, R), generator=gen).numpy()
    q = torch.randn(B, T, R, bits, generator=gen, dtype=torch.float64)
    grad = torch.randn(B, T, R, D, generator=gen, dtype=torch.float64)
    vt = np.ones((B, T), bool)
    vt[1, order] = False
    valid = om.valid_mask(order, B, T, valid_tokens=vt)
    rows = om.route_rows(codes, [order], bits, 0, R, valid_tokens=vt)[..., 0]
    rows = np.where(rows >= 0, rows + rs * A ** order, -1)
    hard = table[torch.from_numpy(rows).clamp_min(0)] * torch.from_numpy(rows >= 0)[..., None].double()
    temp, scale = 1.3, 0.6
    p = torch.sigmoid(temp * q)
    want = torch.zeros(B, T, R, bits, dtype=torch.float64)
    for b in range(B):
        for t in range(T):
            for r in range(R):
                for e in range(order):
                    w = t - e
                    if w < 0 or w > T - order or not valid[b, w + order - 1]:
                        continue
                    for k in range(bits):
                        want[b, t, r, k] += v[rs + r, e * bits + k] @ grad[b, w + order - 1, r]
    want *= scale * temp * p * (1 - p)
    approx = om.surrogate_grad(grad, hard, q, codes, table, valid, order, bits, rs, temp, scale, False)
    exact = om.surrogate_grad(grad, hard, q, codes, table, valid, order, bits, rs, temp, scale, True)
    assert om.rel_err(approx, want) < 1e-12
    assert om.rel_err(exact, want) < 1e-12


def test_degenerate_cases_are_zero():
    x = case_inputs(recipe.SURROGATE_CASES[0])
    args = (x["grad"], x["hard"], x["q"], x["codes"], x["table"], x["valid"], 2, 4, 1)
    assert om.surrogate_grad(*args, 0.0, 1.0, False).abs().max() == 0
    assert om.surrogate_grad(*args, 1.0, 0.0, True).abs().max() == 0
    short = om.surrogate_grad(x["grad"][:, :1], x["hard"][:, :1], x["q"][:, :1], x["codes"][:, :1], x["table"],
                              x["valid"][:, :1], 2, 4, 1, 1.0, 1.0, False)
    assert short.shape == (2, 1, 3, 4) and short.abs().max() == 0
