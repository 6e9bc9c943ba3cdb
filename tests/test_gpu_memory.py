"""Parity of the memory-layer forward (``LngramMemory``) against the oracle (GPU).

- tiny fp32 layer (d 128, R 8): whole forward within 1e-5 (norm-relative) of the fp64 oracle;
- SB shape bf16 (d 1024, R 184): the fused gather+readout path within 2e-2 of the
  reference-rounding bf16 oracle and of the fp64 oracle, given identical codes; the
  fused and the materialised GPU paths agree;
- full SB size (8 x 2048): router codes bit-exact outside the near-tie band, and the
  output at sampled positions equals the oracle evaluated on the position's causal
  window (2 code lags + 9 conv lags), so the check is exact at any sequence length.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from lngram_hip import ops, workloads
from oracle import memory as om

pytestmark = pytest.mark.gpu

TAU = 2e-5  # near-tie band for code comparisons (router logits with |q| <= TAU may flip sign)


def cfg_of(w: workloads.MemoryWorkload) -> om.MemCfg:
    return om.MemCfg(w.d_model, w.routes, w.mem_dim, w.q_heads, w.kv_heads, w.head_dim, eps=w.norm_eps)


def oracle_params(mem) -> dict:
    sd = {k: v.detach().cpu() for k, v in mem.state_dict().items()}
    out = {k[len("module."):]: v for k, v in sd.items() if k.startswith("module.")}
    out["router.weight"] = sd["router.weight"]
    return out


def codes_check(codes_gpu: np.ndarray, q64: np.ndarray, bits: int = 4):
    want = om.pack_route_codes(q64, bits)
    clear = (np.abs(q64) > TAU).reshape(*q64.shape[:-1], -1, bits).all(-1)
    assert (codes_gpu[clear] == want[clear]).all()
    assert (codes_gpu != want).mean() < 1e-3
    return want, int((~clear).sum())


def test_tiny_fp32_layer(dev):
    w = workloads.TINY
    mem = workloads.build_memory(w, seed=0, device=dev)
    h = workloads.make_hidden(w, seed=1, device=dev)
    h_norm = ops.rmsnorm(h, torch.ones(w.d_model, device=dev), w.norm_eps)
    out = mem(h, h_norm).cpu()
    p = oracle_params(mem)
    cfg = cfg_of(w)
    q64 = om.router_logits(h_norm.cpu(), p["router.weight"]).numpy()
    _, codes_gpu = mem.route_codes(h_norm)
    codes, _ = codes_check(codes_gpu.cpu().numpy().astype(np.int32), q64)
    # given identical codes, the fp32 forward is within 1e-5 of fp64 (and of the fp32 reference path)
    out_given = mem.module(h, torch.as_tensor(codes, device=dev)).cpu()
    ref64 = om.memory_forward(p, cfg, h.cpu().double(), codes)
    ref32 = om.memory_forward(p, cfg, h.cpu(), codes)
    assert om.rel_err(out_given, ref64) < 1e-5
    assert om.rel_err(out_given, ref32) < 1e-5
    assert om.rel_err(out, ref64) < 1e-5  # with the GPU's own codes


def test_sb_shape_fused_bf16(dev):
    w = workloads.SB.with_shape(2, 40)
    mem = workloads.build_memory(w, seed=0, device=dev)
    m = mem.module
    h = workloads.make_hidden(w, seed=3, device=dev)
    h_norm = ops.rmsnorm(h, torch.ones(w.d_model, device=dev, dtype=w.dtype), w.norm_eps)
    p = oracle_params(mem)
    cfg = cfg_of(w)
    q64 = om.router_logits(h_norm.cpu(), p["router.weight"]).numpy()
    _, codes_gpu = mem.route_codes(h_norm)
    codes, _ = codes_check(codes_gpu.cpu().numpy().astype(np.int32), q64)
    ct = torch.as_tensor(codes, device=dev)
    assert m._fused_shape_ok(h)
    fused = m(h, ct).cpu()
    # materialised GPU path (same kernels as decode): gather, project, sink attention, finish
    q = m._project_query(h)
    key, val = m._project_memory(m._lookup_route_chunk(ct, None, 0, m.num_routes, None, None))
    mat = m._finish(m._manual_gqa(q, key, val), None).cpu()
    ref_bf16 = om.memory_forward(p, cfg, h.cpu(), codes)
    ref64 = om.memory_forward(p, cfg, h.cpu().double(), codes)
    assert om.rel_err(fused, ref_bf16) < 2e-2
    assert om.rel_err(fused, ref64) < 2e-2
    assert om.rel_err(mat, ref_bf16) < 2e-2
    assert om.rel_err(fused, mat) < 2e-2


def _window_oracle(p, cfg, h, codes, b, t):
    lo = max(0, t - 11)
    hw = h[b:b + 1, lo:t + 1]
    cw = codes[b:b + 1, lo:t + 1]
    # positions lo, lo+1 of the window lose their n-gram history, but position t only depends on
    # heads at t-9..t, whose windows reach back to t-11 >= lo (or to the true sequence start)
    return om.memory_forward(p, cfg, hw, cw)[0, -1]


def test_sb_full_size_codes_and_sampled_positions(dev):
    w = workloads.SB  # 8 x 2048, R 184
    mem = workloads.build_memory(w, seed=0, device=dev)
    h = workloads.make_hidden(w, seed=4, device=dev)
    h_norm = ops.rmsnorm(h, torch.ones(w.d_model, device=dev, dtype=w.dtype), w.norm_eps)
    out = mem(h, h_norm)
    assert out.shape == (8, 2048, 1024) and bool(torch.isfinite(out).all())
    p = oracle_params(mem)
    cfg = cfg_of(w)
    hn = h_norm.cpu()
    q64 = om.router_logits(hn.reshape(-1, w.d_model), p["router.weight"]).numpy().reshape(8, 2048, -1)
    _, codes_gpu = mem.route_codes(h_norm)
    codes_gpu = codes_gpu.cpu().numpy().astype(np.int32)
    codes, near = codes_check(codes_gpu, q64)
    print(f"near-tie routes at SB size: {near} of {codes.size}")
    # outputs at sampled positions given the oracle's codes
    out_given = mem.module(h, torch.as_tensor(codes, device=dev)).cpu()
    hc = h.cpu()
    rng = np.random.default_rng(0)
    picks = [(0, 0), (0, 1), (0, 2), (3, 9), (7, 2047)] + [(int(rng.integers(0, 8)), int(rng.integers(0, 2048)))
                                                          for _ in range(11)]
    got = torch.stack([out_given[b, t] for b, t in picks])
    want = torch.stack([_window_oracle(p, cfg, hc, codes, b, t) for b, t in picks])
    want64 = torch.stack([om.memory_forward(p, cfg, hc[b:b + 1, max(0, t - 11):t + 1].double(),
                                            codes[b:b + 1, max(0, t - 11):t + 1])[0, -1] for b, t in picks])
    assert om.rel_err(got, want) < 2e-2
    assert om.rel_err(got, want64) < 2e-2


def test_fused_edge_routes_and_short_sequences(dev):
    # R not a multiple of 32 (181 = 5*32 + 21) and T < 3 (all-zero 3-gram rows)
    for routes, b, t in ((181, 3, 2), (33, 1, 7), (200, 1, 1)):
        w = workloads.MemoryWorkload("edge", 1024, routes, 128, 16, 4, 64, b, t, torch.bfloat16)
        mem = workloads.build_memory(w, seed=routes, device=dev)
        m = mem.module
        h = workloads.make_hidden(w, seed=5, device=dev)
        codes = np.random.default_rng(routes).integers(0, 16, (b, t, routes))
        got = m(h, torch.as_tensor(codes, device=dev)).cpu()
        ref64 = om.memory_forward(oracle_params(mem), cfg_of(w), h.cpu().double(), codes)
        assert om.rel_err(got, ref64) < 2e-2
