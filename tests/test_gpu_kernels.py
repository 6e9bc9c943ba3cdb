"""Parity of the individual gfx950 kernels against the oracle (GPU).

Integer work is compared bit-exactly; floating-point work against the fp64 / reference-
rounding oracle with the tolerance written in each test.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from lngram_hip import ops
from oracle import cint
from oracle import memory as om

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().numpy()


# ----------------------------------------------------------------------------- K2: addresses, rows, gather
@pytest.mark.parametrize("cdt", [torch.uint8, torch.int32, torch.int64])
def test_ngram_address_bit_exact(dev, cdt):
    rng = np.random.default_rng(0)
    codes = rng.integers(0, 16, (3, 37, 11))
    for order in (1, 2, 3):
        got = ops.ngram_address(torch.as_tensor(codes).to(cdt).to(dev), order, 4)
        np.testing.assert_array_equal(_np(got), om.ngram_address(codes, order, 4))
    # reference KAT (tests/test_index_layout.py:28-33)
    kat = torch.tensor([[[3], [5], [7], [9]]], dtype=cdt, device=dev)
    assert int(ops.ngram_address(kat, 2, 4)[0, 0, 0]) == 3 + 16 * 5
    assert int(ops.ngram_address(kat, 3, 4)[0, 1, 0]) == 5 + 16 * 7 + 256 * 9
    assert ops.ngram_address(kat[:, :1], 2, 4).shape == (1, 0, 1)


def test_ngram_rows_bit_exact_with_segments(dev):
    rng = np.random.default_rng(1)
    b, t, r = 4, 29, 184
    codes = rng.integers(0, 16, (b, t, r))
    seg = np.cumsum(rng.random((b, t)) < 0.15, axis=1).astype(np.int32)
    valid = rng.random((b, t)) < 0.85
    ct = torch.as_tensor(codes, dtype=torch.uint8, device=dev)
    for s, v in ((None, None), (seg, None), (None, valid), (seg, valid)):
        got = ops.ngram_rows(ct, (2, 3), 4, 0, r, None if s is None else torch.as_tensor(s, device=dev),
                             None if v is None else torch.as_tensor(v, device=dev))
        want = cint.ngram_rows(codes, (2, 3), 4, s, v)
        np.testing.assert_array_equal(_np(got), want)
    got = ops.ngram_rows(ct, (2, 3), 4, 17, 60)
    np.testing.assert_array_equal(_np(got), om.route_rows(codes, (2, 3), 4, 17, 60))


@pytest.mark.parametrize("tdt", [torch.float32, torch.bfloat16, torch.float16])
def test_route_tokens_bit_exact(dev, tdt):
    rng = np.random.default_rng(2)
    b, t, r, md = 2, 13, 9, 32
    codes = rng.integers(0, 16, (b, t, r))
    tables = {n: (torch.randn(r * 16 ** n, md) * 0.02).to(tdt) for n in (2, 3)}
    seg = np.cumsum(rng.random((b, t)) < 0.2, axis=1).astype(np.int32)
    ct = torch.as_tensor(codes, dtype=torch.int32, device=dev)
    tl = [tables[2].to(dev), tables[3].to(dev)]
    cases = [dict(), dict(route_start=2, route_end=7), dict(segment_ids=seg), dict(target_length=3),
             dict(valid_tokens=rng.random((b, t)) < 0.7)]
    for kw in cases:
        dkw = {k: (torch.as_tensor(v, device=dev) if isinstance(v, np.ndarray) else v) for k, v in kw.items()}
        got = ops.route_tokens(ct, tl, (2, 3), 4, **dkw)
        want = om.route_tokens(tables, codes, (2, 3), 4, **kw)
        assert got.dtype == tdt
        np.testing.assert_array_equal(_np(got.float()), want.float().numpy())


def test_route_tokens_sb_width_and_odd_width(dev):
    rng = np.random.default_rng(3)
    for md in (128, 3):  # 256-byte rows (vector path) and 6-byte rows (2-byte path)
        r = 5
        codes = rng.integers(0, 16, (1, 9, r))
        tables = {n: torch.randn(r * 16 ** n, md).to(torch.bfloat16) for n in (2, 3)}
        got = ops.route_tokens(torch.as_tensor(codes, device=dev), [tables[2].to(dev), tables[3].to(dev)], (2, 3), 4)
        want = om.route_tokens(tables, codes, (2, 3), 4)
        np.testing.assert_array_equal(_np(got.float()), want.float().numpy())


def test_empty_and_short_sequences(dev):
    tab = [torch.zeros(4 * 256, 8, device=dev), torch.zeros(4 * 4096, 8, device=dev)]
    out = ops.route_tokens(torch.zeros(2, 0, 4, dtype=torch.uint8, device=dev), tab, (2, 3), 4)
    assert out.shape == (2, 0, 4, 16)
    out = ops.route_tokens(torch.ones(1, 1, 4, dtype=torch.uint8, device=dev), tab, (2, 3), 4)
    assert out.shape == (1, 1, 4, 16) and float(out.abs().max()) == 0


# ----------------------------------------------------------------------------- K1: router + codes
def test_pack_route_codes_bit_exact(dev):
    q = torch.randn(57, 4 * 23)
    q[0, :8] = torch.tensor([0.0, -0.0, float("nan"), 1e-30, -1e-30, 5.0, -5.0, 0.0])
    got = ops.pack_route_codes(q.to(dev), 4)
    np.testing.assert_array_equal(_np(got), cint.pack_codes(q.numpy(), 4))
    assert _np(got)[0, :2].tolist() == [8, 2]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(300, 1024, 736), (37, 128, 32), (129, 2304, 724), (4500, 1024, 736),
                                   (4100, 2304, 724), (4200, 1056, 736)])
def test_router_logits_and_codes(dev, dtype, shape):
    m, k, n = shape
    g = torch.Generator().manual_seed(m + k)
    x = torch.randn(m, k, generator=g).to(dtype)
    w = (torch.randn(n, k, generator=g) * 0.02).to(dtype)
    q64 = om.router_logits(x, w).numpy()
    logits, codes = ops.router_codes(x.to(dev), w.to(dev), 4, want_logits=True, codes_dtype=torch.uint8)
    # fp32 accumulation error bound: |err| <= K * 2^-24 * sum|x w|  (tolerance written here)
    bound = k * 2.0 ** -24 * (x.double().abs() @ w.double().abs().T).numpy()
    assert (np.abs(_np(logits) - q64) <= bound + 1e-12).all()
    want = om.pack_route_codes(q64, 4)
    tau = 2e-5  # near-tie band: codes compared bit-exactly where every bit's |q| > tau
    clear = (np.abs(q64) > tau).reshape(m, n // 4, 4).all(-1)
    got = _np(codes).astype(np.int32)
    assert (got[clear] == want[clear]).all()
    assert (got != want).mean() < 1e-3
    _, codes_only = ops.router_codes(x.to(dev), w.to(dev), 4, want_logits=False, codes_dtype=torch.int32)
    np.testing.assert_array_equal(_np(codes_only), got)


def test_router_codes_two_bit_routes_large(dev):
    # bits != 4 at a large batch: fp32 logits from the wide-tile MFMA kernel, then the pack kernel
    m, k, n = 4500, 1024, 736
    g = torch.Generator().manual_seed(7)
    x = torch.randn(m, k, generator=g).bfloat16()
    w = (torch.randn(n, k, generator=g) * 0.02).bfloat16()
    q64 = om.router_logits(x, w).numpy()
    logits, codes = ops.router_codes(x.to(dev), w.to(dev), 2, want_logits=True, codes_dtype=torch.int32)
    bound = k * 2.0 ** -24 * (x.double().abs() @ w.double().abs().T).numpy()
    assert (np.abs(_np(logits) - q64) <= bound + 1e-12).all()
    np.testing.assert_array_equal(_np(codes), om.pack_route_codes(_np(logits).astype(np.float64), 2))


# ----------------------------------------------------------------------------- K3 pieces
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("dim", [1024, 200])
def test_rmsnorm(dev, dtype, fused, dim):
    # model.RMSNorm (two roundings) and lngram_v2.RMSNorm (F.rms_norm, one rounding): the golden
    # fixtures pin both oracle forms to the reference; the kernel may differ from them only where
    # its sum of squares (another summation order) moves a value across a rounding boundary
    x = torch.randn(33, dim).to(dtype)
    w = (1 + 0.1 * torch.randn(dim)).to(dtype)
    got = ops.rmsnorm(x.to(dev), w.to(dev), 1e-5, fused=fused).cpu()
    want = (om.rms_norm_v2 if fused else om.rms_norm)(x, w, 1e-5)
    if dtype == torch.float32:
        torch.testing.assert_close(got, want, rtol=1e-6, atol=1e-6)
    else:
        diff = (got.float() - want.float()).abs()
        assert diff.max() <= 2 ** -7 * want.float().abs().max()
        assert (diff > 0).float().mean() < 0.01


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 1e-2)])
@pytest.mark.parametrize("mnk", [(513, 1024, 1024), (7, 33, 64), (130, 256, 256), (4100, 1000, 1024),
                                 (8192, 1024, 96)])
def test_linear(dev, dtype, tol, mnk):
    m, n, k = mnk
    x = torch.randn(m, k).to(dtype)
    w = (torch.randn(n, k) * 0.05).to(dtype)
    got = ops.linear(x.to(dev), w.to(dev)).cpu()
    want = x.double() @ w.double().T
    assert om.rel_err(got, want) < tol


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
def test_sink_attention_and_probabilities(dev, dtype, tol):
    cfg = om.MemCfg(1024, 184, 128, 16, 4, 64)
    b, t = 2, 5
    q = torch.randn(b, t, cfg.q_heads, cfg.head_dim).to(dtype)
    kv = torch.randn(b, t, cfg.routes, 2 * cfg.kv_heads * cfg.head_dim).to(dtype)
    kh = cfg.kv_heads * cfg.head_dim
    key = kv[..., :kh].view(b, t, cfg.routes, cfg.kv_heads, cfg.head_dim).permute(0, 1, 3, 2, 4)
    val = kv[..., kh:].view(b, t, cfg.routes, cfg.kv_heads, cfg.head_dim).permute(0, 1, 3, 2, 4)
    want = om.manual_gqa(cfg, q, key, val)
    ref64 = om.manual_gqa(cfg, q.double(), key.double(), val.double())
    kvd = kv.to(dev)
    keyd = kvd[..., :kh].view(b, t, cfg.routes, cfg.kv_heads, cfg.head_dim).permute(0, 1, 3, 2, 4)
    vald = kvd[..., kh:].view(b, t, cfg.routes, cfg.kv_heads, cfg.head_dim).permute(0, 1, 3, 2, 4)
    got = ops.sink_attention(q.to(dev).view(b, t, cfg.kv_heads, cfg.groups, cfg.head_dim), keyd, vald,
                             cfg.softmax_scale, cfg.sink_logit).reshape(b, t, cfg.q_heads, cfg.head_dim).cpu()
    assert om.rel_err(got, want) < tol
    assert om.rel_err(got, ref64) < tol
    scores = torch.randn(40, 184) * 3
    p = ops.sink_probabilities(scores.to(dev), cfg.sink_logit).cpu()
    torch.testing.assert_close(p.double(), om.sink_probabilities(scores.double(), cfg.sink_logit), rtol=1e-5,
                               atol=1e-7)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
def test_causal_conv(dev, dtype, tol):
    cfg = om.MemCfg(256, 4, 16, 4, 2, 64)
    p = {"short_conv.norm.weight": 1 + 0.1 * torch.randn(256), "short_conv.conv.weight": 0.2 * torch.randn(256, 1, 4)}
    mixed = (torch.randn(3, 37, 256) * 0.01).to(dtype)
    want = mixed + om.causal_conv(p, cfg, mixed)
    ref64 = mixed.double() + om.causal_conv(p, cfg, mixed.double())
    got = ops.causal_conv(mixed.to(dev), p["short_conv.norm.weight"].to(dev), p["short_conv.conv.weight"].to(dev),
                          3, cfg.eps).cpu()
    assert om.rel_err(got, want) < tol and om.rel_err(got, ref64) < tol
    # the reference's rounding sequence (F.rms_norm, one rounding), not just its tolerance
    assert om.rel_err(got, want) < tol / 10
    got2 = ops.causal_conv(mixed.to(dev), p["short_conv.norm.weight"].to(dev), p["short_conv.conv.weight"].to(dev),
                           3, cfg.eps, residual=False).cpu()
    assert om.rel_err(got2, ref64 - mixed.double()) < tol


@pytest.mark.parametrize("b,t,d,k", [(2, 300, 1024, 1024), (3, 37, 1000, 64), (1, 5, 8, 32), (2, 70, 2048, 64)])
def test_linear_rowsq_and_conv_from_row_stats(dev, b, t, d, k):
    # o_proj with fused row statistics, then the conv that consumes them: the statistics are the
    # sums of squares of the bf16 outputs, the conv matches the oracle with the reference rounding
    g = torch.Generator().manual_seed(d + t)
    x = torch.randn(b, t, k, generator=g).to(torch.bfloat16)
    w = (torch.randn(d, k, generator=g) * 0.05).to(torch.bfloat16)
    y, rowsq = ops.linear_rowsq(x.to(dev), w.to(dev))
    y, rowsq = y.cpu(), rowsq.cpu()
    assert om.rel_err(y, x.double() @ w.double().T) < 1e-2
    assert rowsq.shape[1] == b * t
    ss = y.double().pow(2).sum(-1).reshape(-1)
    torch.testing.assert_close(rowsq.double().sum(0), ss, rtol=1e-5, atol=1e-6)
    cfg = om.MemCfg(d, 4, 16, 4, 2, 64)
    p = {"short_conv.norm.weight": 1 + 0.1 * torch.randn(d, generator=g),
         "short_conv.conv.weight": 0.2 * torch.randn(d, 1, 4, generator=g)}
    nw, cw = p["short_conv.norm.weight"].to(dev), p["short_conv.conv.weight"].to(dev)
    got = ops.causal_conv_rowsq(y.to(dev), rowsq.to(dev), nw, cw, 3, cfg.eps).cpu()
    want = y + om.causal_conv(p, cfg, y)
    ref64 = y.double() + om.causal_conv(p, cfg, y.double())
    assert om.rel_err(got, want) < 2e-2 and om.rel_err(got, ref64) < 2e-2
    # same kernel inputs through the self-normalising conv: equal up to the summation order
    other = ops.causal_conv(y.to(dev), nw, cw, 3, cfg.eps).cpu()
    assert om.rel_err(got, other) < 8e-3
    with pytest.raises(RuntimeError):
        ops.causal_conv_rowsq(y.to(dev), rowsq.to(dev), nw, cw, 2, cfg.eps)


@pytest.mark.parametrize("m,n,k", [(4096, 1024, 1024), (1280, 200, 128)])
def test_linear_rowscale(dev, m, n, k):
    # the query projection with the RMSNorm row scale formed inside the GEMM
    # (_project_query, lngram_v2.py:1115-1118, the norm weight folded into w): against fp64, and
    # against the plain projection scaled afterwards
    g = torch.Generator().manual_seed(m + n)
    x = (torch.randn(m, k, generator=g) * 0.7).bfloat16()
    x[3] = 0                                   # a zero row: scale rsqrt(eps)
    w = (torch.randn(n, k, generator=g) * 0.03).bfloat16()
    eps = 1e-5
    assert ops.linear_rowscale_ok(x.to(dev), w.to(dev))
    got = ops.linear_rowscale(x.to(dev), w.to(dev), eps).cpu()
    xd = x.double()
    ref = (xd @ w.double().T) * torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + eps)
    assert om.rel_err(got, ref) < 1e-2
    assert float((got.double() - ref).abs().max()) <= float(ref.abs().max()) * 2 ** -7
    plain = ops.linear(x.to(dev), w.to(dev)).cpu().float()
    scaled = plain * torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + eps)
    assert float((got.float() - scaled).abs().max()) <= float(scaled.abs().max()) * 2 ** -6
    assert not ops.linear_rowscale_ok(x[:512].to(dev), w.to(dev))
    with pytest.raises(RuntimeError):
        ops.linear_rowscale(x[:512].to(dev), w.to(dev), eps)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
def test_causal_conv_generic_shape(dev, dtype, tol):
    # kernel 3, dilation 2, odd width: the general (non-specialised) conv kernel
    cfg = om.MemCfg(100, 4, 16, 4, 2, 25, orders=(2,), conv_kernel=3)
    p = {"short_conv.norm.weight": 1 + 0.1 * torch.randn(100), "short_conv.conv.weight": 0.2 * torch.randn(100, 1, 3)}
    mixed = (torch.randn(2, 21, 100) * 0.01).to(dtype)
    ref64 = mixed.double() + om.causal_conv(p, cfg, mixed.double())
    got = ops.causal_conv(mixed.to(dev), p["short_conv.norm.weight"].to(dev), p["short_conv.conv.weight"].to(dev),
                          cfg.conv_dilation, cfg.eps).cpu()
    assert om.rel_err(got, ref64) < tol


# ----------------------------------------------------------------------------- K4: scan
@pytest.mark.parametrize("b,t,n", [(8, 4096, 256), (3, 301, 16), (2, 1, 8), (1, 64, 64), (1, 65, 70)])
def test_ssm_scan(dev, b, t, n):
    g = torch.Generator().manual_seed(t)
    a = 0.9 + 0.099 * torch.rand(n, generator=g)
    u = torch.randn(b, t, n, generator=g)
    s0 = torch.randn(b, n, generator=g)
    for init in (None, s0):
        got = ops.ssm_scan(a.to(dev), u.to(dev), None if init is None else init.to(dev)).cpu().numpy()
        want = om.ssm_scan(a.numpy(), u.numpy(), None if init is None else init.numpy())
        assert np.abs(got - want).max() < 1e-5 * max(1.0, np.abs(want).max())  # 1e-5 (fp32 tolerance)


def test_ssm_scan_workspace_reuse_across_shapes(dev):
    # one workspace across calls of different shapes (larger, smaller, channel groups of 256 and a
    # width that is not a multiple of 4): every call equals the recurrence, so the in-kernel reset
    # of the counters and the epoch-tagged flags leave nothing stale behind
    g = torch.Generator().manual_seed(5)
    for b, t, n in ((2, 1000, 300), (8, 4096, 256), (1, 130, 7), (3, 257, 512), (8, 4096, 256), (1, 1, 4)):
        a = 0.5 + 0.499 * torch.rand(n, generator=g)
        u = torch.randn(b, t, n, generator=g)
        s0 = torch.randn(b, n, generator=g)
        got = ops.ssm_scan(a.to(dev), u.to(dev), s0.to(dev)).cpu().numpy()
        want = om.ssm_scan(a.numpy(), u.numpy(), s0.numpy())
        assert np.abs(got - want).max() < 1e-5 * max(1.0, np.abs(want).max()), (b, t, n)


def test_ssm_scan_direct_carry_when_waits_run_out(dev):
    # the host bounds every tile's wait for its predecessors' records at zero sleeps: a tile whose
    # predecessors have not yet published forms its carry from u directly.  Every kernel exits
    # normally and the states still equal the recurrence; the status word says whether the direct
    # path ran (bit 0) and reads back as zero after a default call.
    g = torch.Generator().manual_seed(11)
    for b, t, n in ((8, 4096, 256), (3, 301, 70)):
        a = 0.9 + 0.099 * torch.rand(n, generator=g)
        u = torch.randn(b, t, n, generator=g)
        s0 = torch.randn(b, n, generator=g)
        ops.ssm_scan_status(dev)
        got = ops.ssm_scan(a.to(dev), u.to(dev), s0.to(dev), spin_limit=0).cpu().numpy()
        want = om.ssm_scan(a.numpy(), u.numpy(), s0.numpy())
        assert np.abs(got - want).max() < 1e-5 * max(1.0, np.abs(want).max()), (b, t, n)
        assert ops.ssm_scan_status(dev) in (0, 1)
        again = ops.ssm_scan(a.to(dev), u.to(dev), s0.to(dev)).cpu().numpy()
        assert np.abs(again - want).max() < 1e-5 * max(1.0, np.abs(want).max()), (b, t, n)
        assert ops.ssm_scan_status(dev) == 0


def test_ssm_scan_constant_input_closed_form(dev):
    a = torch.tensor([0.9, 0.95, 0.999, 0.5])
    u = torch.tensor([1.0, -2.0, 0.5, 3.0])
    got = ops.ssm_scan(a.to(dev), u.expand(1, 1000, 4).contiguous().to(dev)).cpu().numpy()[0]
    want = om.ssm_scan_closed_form_constant(a.numpy(), u.numpy(), 1000)
    assert np.abs(got - want).max() < 1e-5


# ----------------------------------------------------------------------------- K5: tree acceptance
PARENT = (-1, 0, 1, 0, 3, 1)


@pytest.mark.parametrize("argmax,path,new", [
    ([3, 9, 9, 4, 8, 9], [0, 3, 4], [3, 4, 8]),     # reference tests/test_live_tree.py:44-52
    ([1, 5, 9, 9, 9, 6], [0, 1, 5], [1, 5, 6]),
    ([9, 9, 9, 9, 9, 9], [0], [9]),
])
def test_tree_accept_known_answers(dev, argmax, path, new):
    toks = [7, 1, 2, 3, 4, 5]
    p, plen, nt = ops.tree_accept(torch.tensor(PARENT, device=dev), torch.tensor(toks, device=dev),
                                  torch.tensor(argmax, device=dev))
    ln = int(plen[0])
    assert _np(p)[:ln].tolist() == path and _np(nt)[:ln].tolist() == new
    assert cint.tree_accept(PARENT, toks, argmax) == (path, new)


def test_tree_accept_random_trees(dev):
    rng = np.random.default_rng(7)
    for _ in range(50):
        n = int(rng.integers(1, 20))
        parent = [-1] + [int(rng.integers(0, i)) for i in range(1, n)]
        toks = rng.integers(0, 4, n).tolist()
        am = rng.integers(0, 4, n).tolist()
        p, plen, nt = ops.tree_accept(torch.tensor(parent, device=dev), torch.tensor(toks, device=dev),
                                      torch.tensor(am, device=dev))
        ln = int(plen[0])
        assert (_np(p)[:ln].tolist(), _np(nt)[:ln].tolist()) == cint.tree_accept(parent, toks, am)


def test_large_linear_and_row_sumsq(dev):
    """Large bf16 projection against fp64, and against the same kernel with the row-statistics
    epilogue (bit for bit); the separate row sums of squares against the epilogue's partials and
    fp64."""
    g = torch.Generator().manual_seed(21)
    x = (torch.randn(4096, 1024, generator=g) * 0.5).bfloat16()
    w = (torch.randn(768, 1024, generator=g) * 0.02).bfloat16()
    y_lt = ops.linear(x.to(dev), w.to(dev))
    y_mf, rsq = ops.linear_rowsq(x.to(dev), w.to(dev))
    ref = x.double() @ w.double().T
    assert om.rel_err(y_lt.cpu().double(), ref) < 1e-2
    assert torch.equal(y_lt, y_mf)
    s = ops.row_sumsq(y_mf)
    want = (y_mf.double() ** 2).sum(-1)
    assert s.shape == (1, 4096)
    torch.testing.assert_close(s[0].double(), want, rtol=1e-5, atol=0)
    torch.testing.assert_close(s[0], rsq.sum(0), rtol=1e-5, atol=0)
