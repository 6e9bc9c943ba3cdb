"""The lookup surrogate's backward on the GPU (``lng_surrogate_grad``, ``lng_table_grad`` and the
mirror's ``_LngramSurrogate`` / training-mode ``_lookup_route_chunk``; reference
``lngram_v2.py:328-464``, ``:1047-1113``).

- The reference's own gradients (``tests/golden/surrogate.npz``): norm-relative < 1e-5.
- The fp64 oracle at larger shapes (mem_dim 32..256, orders 1..3, 1..4-bit codes, fp32 and bf16
  tables, bf16 logits and gradient outputs): < 1e-5 (bf16 outputs: the bf16 rounding).
- At the full SB shape (8 x 2048 tokens, 184 routes, mem_dim 128, bf16, orders 2 and 3), a table
  linear in the address bits with small-integer entries and gradients: every dot product is
  exact in fp32, so the kernel must equal the closed form up to the fp32 slope (< 1e-6).
- The table gradient against an fp64 scatter, and the training-mode lookup end to end.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from lngram_hip import ops
from oracle import memory as om

GOLD = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLD))
import recipe  # noqa: E402
from .test_oracle_surrogate import case_inputs  # noqa: E402

pytestmark = pytest.mark.gpu


def _gold() -> dict:
    with np.load(GOLD / "surrogate.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("case", recipe.SURROGATE_CASES, ids=[c[0] for c in recipe.SURROGATE_CASES])
def test_kernel_matches_reference_gradients(dev, case):
    name, order, bits, R, rs, B, T, D, dt_name, temp, scale, exact = case
    x = case_inputs(case)
    g = _gold()
    got = ops.surrogate_grad(x["grad"].to(dev), x["hard"].to(dev), x["q"].to(dev),
                             torch.from_numpy(x["codes"]).to(dev), x["table"].to(dev),
                             torch.from_numpy(x["valid"]).to(dev), order, bits, rs, temp, scale, exact)
    assert got.dtype == torch.float32 and got.shape == (B, T, R, bits)
    want = torch.from_numpy(g[f"{name}_grad_q"])
    assert om.rel_err(got.cpu(), want) < 1e-5
    ora = om.surrogate_grad(x["grad"], x["hard"], x["q"], x["codes"], x["table"], x["valid"], order, bits, rs, temp,
                            scale, exact)
    assert om.rel_err(got.cpu(), ora) < 1e-5


def _random_case(seed, B, T, R, rs, D, order, bits, dtype, q_dtype=torch.float32, invalid=True):
    gen = torch.Generator().manual_seed(seed)
    A = 1 << bits
    table = (torch.randn((rs + R) * A ** order, D, generator=gen) * 0.5).to(dtype)
    codes = torch.randint(0, A, (B, T, R), generator=gen)
    q = torch.randn(B, T, R, bits, generator=gen).to(q_dtype)
    grad = torch.randn(B, T, R, D, generator=gen).to(dtype)
    vt = np.ones((B, T), bool)
    if invalid and T > order + 2:
        vt[B - 1, order + 1] = False
    valid = om.valid_mask(order, B, T, valid_tokens=vt)
    rows = om.route_rows(codes.numpy(), [order], bits, 0, R, valid_tokens=vt)[..., 0]
    rows = np.where(rows >= 0, rows + rs * A ** order, -1)
    hard = table[torch.from_numpy(rows).clamp_min(0)] * torch.from_numpy(rows >= 0)[..., None].to(dtype)
    return dict(table=table, codes=codes, q=q, grad=grad, valid=valid, hard=hard)


@pytest.mark.parametrize("D,order,bits,dtype", [(128, 3, 4, torch.bfloat16), (128, 2, 4, torch.bfloat16),
                                                (256, 2, 3, torch.float32), (64, 1, 4, torch.float32),
                                                (32, 3, 2, torch.bfloat16)])
@pytest.mark.parametrize("exact", [False, True])
def test_kernel_matches_oracle(dev, D, order, bits, dtype, exact):
    B, T, R, rs = 2, 37, 6, 3
    x = _random_case(D + order + bits, B, T, R, rs, D, order, bits, dtype)
    temp, scale = 0.9, 1.1
    got = ops.surrogate_grad(x["grad"].to(dev), x["hard"].to(dev), x["q"].to(dev), x["codes"].to(dev),
                             x["table"].to(dev), torch.from_numpy(x["valid"]).to(dev), order, bits, rs, temp, scale,
                             exact)
    want = om.surrogate_grad(x["grad"], x["hard"], x["q"], x["codes"].numpy(), x["table"], x["valid"], order, bits,
                             rs, temp, scale, exact)
    assert want.abs().max() > 0
    assert om.rel_err(got.cpu(), want) < 1e-5


def test_bf16_logits_give_bf16_gradient_and_codes_any_int_dtype(dev):
    B, T, R, rs, D, order, bits = 1, 20, 4, 0, 128, 3, 4
    x = _random_case(5, B, T, R, rs, D, order, bits, torch.bfloat16, q_dtype=torch.bfloat16)
    want = om.surrogate_grad(x["grad"], x["hard"], x["q"], x["codes"].numpy(), x["table"], x["valid"], order, bits,
                             rs, 1.0, 1.0, False)
    outs = []
    for cdt in (torch.uint8, torch.int32, torch.int64):
        got = ops.surrogate_grad(x["grad"].to(dev), x["hard"].to(dev), x["q"].to(dev), x["codes"].to(cdt).to(dev),
                                 x["table"].to(dev), torch.from_numpy(x["valid"]).to(dev), order, bits, rs, 1.0, 1.0,
                                 False)
        assert got.dtype == torch.bfloat16
        outs.append(got)
        assert om.rel_err(got.float().cpu(), want) < 5e-3
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


def test_degenerate_and_errors(dev):
    x = _random_case(9, 1, 2, 2, 0, 32, 3, 4, torch.float32)
    args = [x["grad"].to(dev), x["hard"].to(dev), x["q"].to(dev), x["codes"].to(dev), x["table"].to(dev),
            torch.from_numpy(x["valid"]).to(dev)]
    assert ops.surrogate_grad(*args, 3, 4, 0, 1.0, 1.0, False).abs().max().item() == 0   # T < order
    y = _random_case(9, 1, 9, 2, 0, 32, 2, 4, torch.float32)
    args = [y["grad"].to(dev), y["hard"].to(dev), y["q"].to(dev), y["codes"].to(dev), y["table"].to(dev),
            torch.from_numpy(y["valid"]).to(dev)]
    assert ops.surrogate_grad(*args, 2, 4, 0, 0.0, 1.0, False).abs().max().item() == 0
    assert ops.surrogate_grad(*args, 2, 4, 0, 1.0, 0.0, True).abs().max().item() == 0
    with pytest.raises(RuntimeError, match="fewer rows"):
        ops.surrogate_grad(*args, 2, 4, 1, 1.0, 1.0, False)              # routes 1..2 need 3 route blocks
    z = _random_case(9, 1, 9, 2, 0, 48, 2, 4, torch.float32)
    with pytest.raises(RuntimeError, match="mem_dim"):
        ops.surrogate_grad(z["grad"].to(dev), z["hard"].to(dev), z["q"].to(dev), z["codes"].to(dev),
                           z["table"].to(dev), None, 2, 4, 0, 1.0, 1.0, False)


def _linear_table(gen, R, order, bits, D, dev):
    """Rows w0[r] + sum_j bit_j(addr) v[r, j] with small integers: exact in bf16."""
    nbit = order * bits
    w0 = torch.randint(-3, 4, (R, D), generator=gen).float()
    v = torch.randint(-2, 3, (R, nbit, D), generator=gen).float()
    addr = torch.arange(1 << nbit)
    ab = ((addr[:, None] >> torch.arange(nbit)) & 1).float()
    table = (w0[:, None, :] + torch.einsum("aj,rjd->rad", ab, v)).reshape(-1, D)
    return table.to(torch.bfloat16).to(dev), v.to(dev)


def test_sb_shape_linear_table_closed_form(dev):
    """Full SB shape: both orders' gradients against the closed form
    G[t, k] = scale * T * p(1-p) * sum_e v[r, e*bits + k] . g[window t - e]."""
    B, T, R, D, bits = 8, 2048, 184, 128, 4
    gen = torch.Generator().manual_seed(2024)
    codes = torch.randint(0, 16, (B, T, R), generator=gen, dtype=torch.uint8).to(dev)
    q = torch.randn(B, T, R, bits, generator=gen).to(dev)
    temp, scale = 1.0, 1.0
    p = torch.sigmoid(temp * q.double())
    for order in (2, 3):
        table, v = _linear_table(gen, R, order, bits, D, dev)
        grad = torch.randint(-2, 3, (B, T, R, D), generator=gen, dtype=torch.int8).to(dev).to(torch.bfloat16)
        valid = torch.ones(B, T, dtype=torch.bool, device=dev)
        valid[:, :order - 1] = False
        hard = ops.route_tokens(codes, [table], [order], bits)
        print(f"surrogate SB order {order}", flush=True)
        got = ops.surrogate_grad(grad, hard, q, codes, table, valid, order, bits, 0, temp, scale, False)
        torch.cuda.synchronize()
        # closed form: window w (ending at w + order - 1) contributes v[r, e*bits+k] . g_w to position w + e
        gw = grad[:, order - 1:].double()                                 # [B, VL, R, D]
        vl = T - order + 1
        want = torch.zeros(B, T, R, bits, dtype=torch.float64, device=dev)
        for e in range(order):
            for k in range(bits):
                want[:, e:e + vl, :, k] += (gw * v[:, e * bits + k].double()[None, None]).sum(-1)
        want *= scale * temp * p * (1 - p)
        assert om.rel_err(got.cpu(), want.cpu()) < 1e-6, order
        del hard, grad, table, got, want


@pytest.mark.parametrize("shape", ["sb_packed", "f32_d64", "bf16_d32"])
def test_hard_rows_from_table_equal_saved_rows(dev, shape):
    """``hard_memory`` None (the kernel reads each window's looked-up row from the table) gives the
    same gradient, bit for bit, as passing the lookup's own rows ``table[row] * valid``: the packed
    bf16 kernel of the SB lookup (mem_dim 128, 4-bit codes, orders 2 and 3) and the generic one, with
    masked positions and a route offset."""
    B, T, R, rs, D, bits, dt, orders = {"sb_packed": (2, 300, 184, 0, 128, 4, torch.bfloat16, (2, 3)),
                                        "f32_d64": (2, 70, 5, 1, 64, 2, torch.float32, (1, 3)),
                                        "bf16_d32": (3, 50, 7, 0, 32, 3, torch.bfloat16, (2,))}[shape]
    gen = torch.Generator().manual_seed(31)
    A = 1 << bits
    for order in orders:
        table = (torch.randn((rs + R) * A ** order, D, generator=gen) * 0.5).to(dt).to(dev)
        codes = torch.randint(0, A, (B, T, R), generator=gen, dtype=torch.uint8).to(dev)
        q = torch.randn(B, T, R, bits, generator=gen).to(dev)
        grad = torch.randn(B, T, R, D, generator=gen).to(dt).to(dev)
        valid = torch.rand(B, T, generator=gen) > 0.2
        valid[:, :order - 1] = False
        valid = valid.to(dev)
        hard = ops.route_tokens(codes, [table[rs * A ** order:]], [order], bits) * valid[:, :, None, None].to(dt)
        for exact in (False, True):
            want = ops.surrogate_grad(grad, hard, q, codes, table, valid, order, bits, rs, 0.7, 1.3, exact)
            got = ops.surrogate_grad(grad, None, q, codes, table, valid, order, bits, rs, 0.7, 1.3, exact)
            assert torch.equal(got, want), (shape, order, exact)


@pytest.mark.parametrize("saved,case", [(False, "uniform"), (True, "uniform"), (False, "skewed")])
def test_order3_binned_path_matches_direct_path_and_oracle(dev, saved, case):
    """Order 3 with a workspace (windows binned by their newest code, a 64 KB sub-block of the
    table on chip per bin) against the direct kernel (fp32 rounding: the within-row summation
    order differs) and the fp64 oracle, with masked positions and a route offset.  "skewed" puts
    about 4,000 of a route's 5,000 windows in one bin: more than one on-chip list holds, so the
    bin is listed in ranges."""
    B, T, R, rs = {"uniform": (3, 400, 40, 2), "skewed": (2, 2500, 6, 1)}[case]
    D, bits, order = 128, 4, 3
    gen = torch.Generator().manual_seed(41)
    A = 1 << bits
    table = (torch.randn((rs + R) * A ** order, D, generator=gen) * 0.5).to(torch.bfloat16)
    codes = torch.randint(0, A, (B, T, R), generator=gen, dtype=torch.uint8)
    if case == "skewed":
        codes[torch.rand(B, T, R, generator=gen) < 0.8] = 3
    q = torch.randn(B, T, R, bits, generator=gen)
    grad = torch.randn(B, T, R, D, generator=gen).to(torch.bfloat16)
    valid = torch.rand(B, T, generator=gen) > 0.15
    valid[:, :order - 1] = False
    hard = ops.route_tokens(codes.to(dev), [table[rs * A ** order:].to(dev)], [order], bits) * \
        valid.to(dev)[:, :, None, None].to(torch.bfloat16)
    args = (grad.to(dev), hard if saved else None, q.to(dev), codes.to(dev), table.to(dev), valid.to(dev), order,
            bits, rs, 0.9, 1.1, False)
    assert ops.lib().lng_surrogate_workspace_bytes(B, T, R, D, order, bits, 1, 0) > 0
    got = ops.surrogate_grad(*args)
    direct = ops.surrogate_grad(*args, workspace=False)
    assert om.rel_err(got.cpu(), direct.cpu()) < 1e-6
    want = om.surrogate_grad(grad, hard.cpu(), q, codes.numpy(), table, valid.numpy(), order, bits, rs, 0.9, 1.1, False)
    assert om.rel_err(got.cpu(), want) < 1e-5
    again = ops.surrogate_grad(*args)                     # the workspace is reused: same result
    assert torch.equal(again, got)
    # the binned path takes at most 65,536 windows a route; longer calls use the direct kernel
    assert ops.lib().lng_surrogate_workspace_bytes(1, 65537, R, D, order, bits, 1, 0) == 0


def test_order3_binned_path_at_its_largest_route(dev):
    """B T = 65,536 windows a route, the most the binned path takes (every thread's four 32-window
    chunks in use, each bin over the 2048-entry list, so every bin is listed in ranges), against
    the direct kernel; one window more and the call takes the direct kernel."""
    B, T, R, rs, D, bits, order = 2, 32768, 3, 1, 128, 4, 3
    gen = torch.Generator().manual_seed(45)
    A = 1 << bits
    table = (torch.randn((rs + R) * A ** order, D, generator=gen) * 0.5).to(torch.bfloat16).to(dev)
    codes = torch.randint(0, A, (B, T, R), generator=gen, dtype=torch.uint8).to(dev)
    q = torch.randn(B, T, R, bits, generator=gen).to(dev)
    grad = torch.randn(B, T, R, D, generator=gen).to(torch.bfloat16).to(dev)
    valid = torch.rand(B, T, generator=gen) > 0.1
    valid[:, :order - 1] = False
    valid = valid.to(dev)
    dt = ops.dtype_code(torch.bfloat16)
    assert ops.lib().lng_surrogate_workspace_bytes(B, T, R, D, order, bits, dt, 0) > 0
    assert ops.lib().lng_surrogate_workspace_bytes(B, T + 1, R, D, order, bits, dt, 0) == 0
    args = (grad, None, q, codes, table, valid, order, bits, rs, 0.9, 1.1, False)
    got = ops.surrogate_grad(*args)
    direct = ops.surrogate_grad(*args, workspace=False)
    assert om.rel_err(got.cpu(), direct.cpu()) < 1e-6


def test_order3_binned_path_takes_the_direct_kernel_for_unaligned_buffers(dev):
    """``lng_surrogate_grad_ws`` through the C ABI with a workspace 16 bytes past a 256-byte boundary,
    then with a gradient buffer 4 bytes past a 16-byte boundary: both calls take the direct kernel
    (the binned path moves 16-byte vectors), so they equal ``lng_surrogate_grad`` bit for bit."""
    B, T, R, rs, D, bits, order = 2, 300, 24, 1, 128, 4, 3
    gen = torch.Generator().manual_seed(43)
    A = 1 << bits
    table = (torch.randn((rs + R) * A ** order, D, generator=gen) * 0.5).to(torch.bfloat16).to(dev)
    codes = torch.randint(0, A, (B, T, R), generator=gen, dtype=torch.uint8).to(dev)
    q = torch.randn(B, T, R, bits, generator=gen).to(dev)
    grad = torch.randn(B, T, R, D, generator=gen).to(torch.bfloat16).to(dev)
    valid = torch.ones(B, T, dtype=torch.bool)
    valid[:, :order - 1] = False
    valid = valid.to(dev)
    lib = ops.lib()
    nws = lib.lng_surrogate_workspace_bytes(B, T, R, D, order, bits, ops.dtype_code(torch.bfloat16), 0)
    assert nws > 0
    want = ops.surrogate_grad(grad, None, q, codes, table, valid, order, bits, rs, 0.9, 1.1, False, workspace=False)
    ws = torch.empty(nws + 512, dtype=torch.uint8, device=dev)
    store = torch.empty(B * T * R * bits + 1, dtype=torch.float32, device=dev)
    for ws_off, out in ((16, store[:-1]), (0, store[1:])):
        out.zero_()
        rc = lib.lng_surrogate_grad_ws(
            grad.data_ptr(), None, ops.dtype_code(grad.dtype), q.data_ptr(), ops.dtype_code(q.dtype), codes.data_ptr(),
            ops.dtype_code(codes.dtype), table.data_ptr(), table.shape[0], valid.data_ptr(), B, T, R, rs, D, order,
            bits, 0.9, 1.1, 0, ws.data_ptr() + ws_off, nws, out.data_ptr(), ops.dtype_code(out.dtype),
            torch.cuda.current_stream(dev).cuda_stream)
        assert rc == 0
        torch.cuda.synchronize()
        assert torch.equal(out.view(B, T, R, bits), want), ws_off


def test_table_grad_matches_scatter(dev):
    B, T, R, rs, D, order, bits = 2, 30, 5, 1, 64, 3, 2
    x = _random_case(17, B, T, R, rs, D, order, bits, torch.float32)
    rows_n = x["table"].shape[0]
    got = ops.table_grad(x["grad"].to(dev), x["codes"].to(dev), torch.from_numpy(x["valid"]).to(dev), order, bits,
                         rs, rows_n)
    rows = om.route_rows(x["codes"].numpy(), [order], bits, 0, R)[..., 0]
    rows = np.where(rows >= 0, rows + rs * (1 << (bits * order)), -1)
    keep = (rows >= 0) & x["valid"][..., None]
    want = torch.zeros(rows_n, D, dtype=torch.float64)
    want.index_add_(0, torch.from_numpy(rows[keep]), x["grad"].double()[torch.from_numpy(keep)])
    assert om.rel_err(got.cpu(), want) < 1e-6


def test_training_lookup_gradients(dev):
    """Training-mode _lookup_route_chunk: route tokens equal the eval lookup; the route logits get
    the sum over orders of the surrogate gradient and the tables the gather gradient."""
    from ffnmem.memory.lngram_v2 import RouteNgramMemoryV2

    torch.manual_seed(0)
    m = RouteNgramMemoryV2(64, bits_per_route=4, num_routes=6, memory_dim=32, ngrams=(2, 3), readout_head_dim=16,
                           readout_num_heads=4, readout_num_kv_heads=2, device=dev, dtype=torch.float32)
    m.q_surrogate_temperature, m.q_surrogate_scale = 0.8, 1.2
    b, t, R = 2, 11, 6
    gen = torch.Generator().manual_seed(1)
    with torch.no_grad():
        for tab in m.tables.values():                   # the default init is zero tables
            tab.weight.copy_(torch.randn(tab.weight.shape, generator=gen))
    q = torch.randn(b, t, R, 4, generator=gen).to(dev).requires_grad_()
    codes = m.quantize_route_logits(q.detach().reshape(b, t, R * 4))
    vt = torch.ones(b, t, dtype=torch.bool, device=dev)
    vt[1, 5] = False
    with torch.no_grad():
        m.eval()
        ref_tokens = m._lookup_route_chunk(codes, None, 0, R, None, vt)
    m.train()
    tokens = m._lookup_route_chunk(codes, q, 0, R, None, vt)
    assert torch.equal(tokens.detach(), ref_tokens)
    w = torch.randn(tokens.shape, generator=gen).to(dev)
    (tokens * w).sum().backward()
    want_q = torch.zeros(b, t, R, 4, dtype=torch.float64)
    for i, n in enumerate(m.ngrams):
        tab = m.tables[f"ngram_{n}"].weight.detach().cpu()
        valid = om.valid_mask(n, b, t, valid_tokens=vt.cpu().numpy())
        g_n = w[..., i * 32:(i + 1) * 32].cpu()
        want_q += om.surrogate_grad(g_n, ref_tokens[..., i * 32:(i + 1) * 32].cpu(), q.detach().cpu(),
                                    codes.cpu().numpy(), tab, valid, n, 4, 0, 0.8, 1.2, False)
        rows = om.route_rows(codes.cpu().numpy(), [n], 4, 0, R, valid_tokens=vt.cpu().numpy())[..., 0]
        keep = rows >= 0
        want_t = torch.zeros(tab.shape, dtype=torch.float64)
        want_t.index_add_(0, torch.from_numpy(rows[keep]), g_n.double()[torch.from_numpy(keep)])
        assert om.rel_err(m.tables[f"ngram_{n}"].weight.grad.cpu(), want_t) < 1e-6
    assert om.rel_err(q.grad.cpu(), want_q) < 1e-5
    with pytest.raises(NotImplementedError, match="backward"):
        m(torch.randn(b, t, 64, device=dev), codes, q_logits=q.reshape(b, t, R * 4))
