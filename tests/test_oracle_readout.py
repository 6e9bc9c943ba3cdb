"""Oracle pinning for the floating-point readout (CPU).

Checks that fix the mathematics independently of the oracle's own formula:
- zero tables give a zero layer output (rows, keys, values and the conv all vanish);
- sink softmax closed form for equal scores (``b0 = ln R``);
- the causal conv's impulse response (tap order, dilation, causality);
- the associativity restatement used by the fused kernel agrees with the reference
  form (keys/values materialised) to fp64 rounding;
- fp32 and bf16 restatements stay within the tolerances of the fp64 one.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import memory as om

CFG = om.MemCfg(d_model=64, routes=5, mem_dim=16, q_heads=4, kv_heads=2, head_dim=16)


def params(cfg: om.MemCfg, seed: int = 0, zero_tables: bool = False) -> dict:
    g = torch.Generator().manual_seed(seed)
    r = lambda *s, std=0.02: torch.randn(*s, generator=g, dtype=torch.float64) * std  # noqa: E731
    p = {
        "readout_query_norm.weight": 1 + r(cfg.d_model, std=0.1),
        "readout_memory_norm.weight": 1 + r(cfg.route_token_dim, std=0.1),
        "readout_q_proj.weight": r(cfg.q_heads * cfg.head_dim, cfg.d_model, std=0.2),
        "readout_kv_proj.weight": r(2 * cfg.kv_heads * cfg.head_dim, cfg.route_token_dim, std=0.2),
        "readout_o_proj.weight": r(cfg.d_model, cfg.q_heads * cfg.head_dim, std=0.2),
        "short_conv.norm.weight": 1 + r(cfg.d_model, std=0.1),
        "short_conv.conv.weight": r(cfg.d_model, 1, cfg.conv_kernel, std=0.3),
        "router.weight": r(cfg.routes * cfg.bits, cfg.d_model, std=0.2),
    }
    for n in cfg.orders:
        t = r(cfg.routes * 16 ** n, cfg.mem_dim, std=1.0)
        p[f"tables.ngram_{n}.weight"] = torch.zeros_like(t) if zero_tables else t
    return p


def test_zero_tables_give_zero_output():
    p = params(CFG, zero_tables=True)
    h = torch.randn(2, 9, CFG.d_model, dtype=torch.float64)
    codes = np.random.default_rng(0).integers(0, 16, (2, 9, CFG.routes))
    out = om.memory_forward(p, CFG, h, codes)
    assert float(out.abs().max()) == 0.0


def test_sink_closed_form_equal_scores():
    r = 7
    b0 = math.log(r)  # sink_initial_active_mass = 0.5
    for s in (-3.0, 0.0, 0.7, 40.0):
        probs = om.sink_probabilities(torch.full((1, r), s, dtype=torch.float64), b0)
        want = 1.0 / (r * (1.0 + math.exp(-s)))
        np.testing.assert_allclose(probs.numpy(), want, rtol=1e-12)
    # zero scores: half the mass on the real routes
    probs = om.sink_probabilities(torch.zeros(1, r, dtype=torch.float64), b0)
    assert abs(float(probs.sum()) - 0.5) < 1e-12


def test_sink_logit_values():
    assert abs(om.MemCfg(1024, 184, 128, 16, 4, 64).sink_logit - math.log(184)) < 1e-15
    assert abs(om.MemCfg(1024, 181, 128, 16, 4, 64).sink_logit - 5.198497031265826) < 1e-12


def test_causal_conv_impulse_response():
    cfg = CFG
    p = params(cfg, seed=3)
    t_len, t0 = 20, 4
    mixed = torch.zeros(1, t_len, cfg.d_model, dtype=torch.float64)
    v = torch.randn(cfg.d_model, dtype=torch.float64)
    mixed[0, t0] = v
    y = om.causal_conv(p, cfg, mixed)
    nw = p["short_conv.norm.weight"]
    xn = v / torch.sqrt(v.pow(2).mean() + cfg.eps) * nw
    w = p["short_conv.conv.weight"][:, 0, :]  # [d, K], taps oldest -> newest
    dil, k = cfg.conv_dilation, cfg.conv_kernel
    for t in range(t_len):
        lag = t - t0
        if lag >= 0 and lag % dil == 0 and lag // dil < k:
            pre = w[:, k - 1 - lag // dil] * xn
            torch.testing.assert_close(y[0, t], torch.nn.functional.silu(pre), rtol=1e-12, atol=1e-12)
        else:
            assert float(y[0, t].abs().max()) == 0.0
    assert dil == 3 and cfg.conv_kernel == 4  # dilation = max n-gram order, left padding 9


def _restructured(p: dict, cfg: om.MemCfg, h: torch.Tensor, codes) -> torch.Tensor:
    """The fused kernel's algebra in fp64 numpy: per token, never materialising keys/values."""
    tables = {n: p[f"tables.ngram_{n}.weight"] for n in cfg.orders}
    tok = om.route_tokens(tables, codes, cfg.orders, cfg.bits).numpy()   # [B,T,R,Dt]
    hn = h.numpy()
    qn = hn / np.sqrt((hn ** 2).mean(-1, keepdims=True) + cfg.eps) * p["readout_query_norm.weight"].numpy()
    q = qn @ p["readout_q_proj.weight"].numpy().T                        # [B,T,H*hd]
    wkv = p["readout_kv_proj.weight"].numpy()
    kh = cfg.kv_heads * cfg.head_dim
    wk, wv = wkv[:kh].reshape(cfg.kv_heads, cfg.head_dim, -1), wkv[kh:].reshape(cfg.kv_heads, cfg.head_dim, -1)
    wm = p["readout_memory_norm.weight"].numpy()
    b, t = h.shape[:2]
    head = np.zeros((b, t, cfg.q_heads, cfg.head_dim))
    for bi in range(b):
        for ti in range(t):
            x = tok[bi, ti]                                               # [R, Dt]
            s = 1.0 / np.sqrt((x ** 2).mean(-1) + cfg.eps)                # [R]
            for hg in range(cfg.q_heads):
                hh = hg // cfg.groups
                qkw = cfg.softmax_scale * wm * (wk[hh].T @ q[bi, ti, hg * cfg.head_dim:(hg + 1) * cfg.head_dim])
                score = s * (x @ qkw)
                m = max(score.max(), cfg.sink_logit)
                e = np.exp(score - m)
                pr = e / (e.sum() + math.exp(cfg.sink_logit - m))
                u = wm * ((pr * s) @ x)
                head[bi, ti, hg] = wv[hh] @ u
    return om.finish(p, cfg, torch.from_numpy(head))


def test_associativity_restatement_matches_reference_form():
    p = params(CFG, seed=5)
    h = torch.randn(2, 7, CFG.d_model, dtype=torch.float64)
    codes = np.random.default_rng(5).integers(0, 16, (2, 7, CFG.routes))
    ref = om.memory_forward(p, CFG, h, codes)
    alt = _restructured(p, CFG, h, codes)
    torch.testing.assert_close(alt, ref, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
def test_reduced_precision_restatements_within_tolerance(dtype, tol):
    p = params(CFG, seed=6)
    h = torch.randn(2, 12, CFG.d_model, dtype=torch.float64)
    codes = np.random.default_rng(6).integers(0, 16, (2, 12, CFG.routes))
    ref = om.memory_forward(p, CFG, h, codes)
    got = om.memory_forward(p, CFG, h, codes, dtype=dtype)
    assert om.rel_err(got, ref) < tol


def test_router_fp64_oracle_is_exact_for_bf16_operands():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, 256, generator=g).to(torch.bfloat16)
    w = (torch.randn(32, 256, generator=g) * 0.02).to(torch.bfloat16)
    q64 = om.router_logits(x, w)
    # bf16 products are exact in fp64; math.fsum gives the correctly rounded sum, so the fp64
    # oracle's only error is its summation order (far below the near-tie band of the tests)
    xi = x.double().numpy()
    wi = w.double().numpy()
    exact = np.array([[math.fsum(xi[m] * wi[n]) for n in range(32)] for m in range(64)])
    np.testing.assert_allclose(q64.numpy(), exact, rtol=0, atol=1e-15)
