"""SD-C memory forward (token-routed memory over a diagonal SSM) against the oracle (GPU).

Pipeline: s = scan(a, u) (fp32) -> router_in = concat(RMSNorm(E[x_{t-1}] or start),
RMSNorm(E[x_t]), s) in bf16 -> router GEMM + sign-pack -> fused gather + readout + finish.
Router features: within one rounding of the feature dtype of the oracle
(``TokenRouterFeatures.forward``, router.py:50-59).  Codes: bit-exact outside the near-tie
band.  Output: 2e-2 norm-relative (bf16) given identical codes.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from lngram_hip import ops, workloads
from oracle import memory as om

from .test_gpu_memory import cfg_of, codes_check, oracle_params

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,d,n,ids", [(torch.bfloat16, 64, 16, True), (torch.bfloat16, 1024, 256, False),
                                           (torch.float32, 32, 0, True), (torch.float32, 48, 8, False),
                                           (torch.float32, 1024, 300, True), (torch.bfloat16, 2560, 8, False)])
def test_router_features_match_oracle(dev, dtype, d, n, ids):
    g = torch.Generator().manual_seed(d + n)
    B, T, V = 3, 17, 50
    table = torch.randn(V, d, generator=g).to(dtype)
    tok = torch.randint(0, V, (B, T), generator=g)
    if ids:
        tok[1, 4] = V + 3                                    # outside the vocabulary: a zero row
    start = (torch.randn(d, generator=g) * 0.02).to(dtype)
    pw = (1 + 0.2 * torch.randn(d, generator=g)).to(dtype)
    cw = (1 + 0.2 * torch.randn(d, generator=g)).to(dtype)
    s = torch.randn(B, T, n, generator=g) if n else None
    emb = table[tok.clamp_max(V - 1)] * (tok < V)[..., None].to(dtype)
    want = om.router_features(emb, start, pw, cw, 1e-5, s)
    kw = dict(ssm_state=None if s is None else s.to(dev))
    if ids:
        got = ops.router_features(table.to(dev), start.to(dev), pw.to(dev), cw.to(dev), 1e-5,
                                  token_ids=tok.to(dev), **kw).cpu()
    else:
        got = ops.router_features(emb.to(dev), start.to(dev), pw.to(dev), cw.to(dev), 1e-5, **kw).cpu()
    assert got.dtype == dtype and got.shape == want.shape
    tol = 4e-3 if dtype == torch.bfloat16 else 2e-6           # one rounding of the feature dtype
    assert om.rel_err(got.double(), want.double()) < tol
    assert (got - want).abs().max() <= tol * want.abs().max()


def _sdc_pipeline(w, dev, seed=0):
    mem = workloads.build_memory(w, seed=seed, device=dev)
    g = torch.Generator().manual_seed(seed + 7)
    E = (torch.randn(w.vocab, w.d_model, generator=g) * 0.02).to(w.dtype)
    tok = torch.randint(0, w.vocab, (w.batch, w.seq), generator=g)
    a = 0.9 + 0.099 * torch.rand(w.ssm_dim, generator=g)
    u = torch.randn(w.batch, w.seq, w.ssm_dim, generator=g)
    h = workloads.make_hidden(w, seed=seed + 1)
    return mem, E, tok, a, u, h


def test_sdc_shape_forward(dev):
    w = workloads.SDC.with_shape(2, 48)
    mem, E, tok, a, u, h = _sdc_pipeline(w, dev)
    feats = mem.router_features
    s = ops.ssm_scan(a.to(dev), u.to(dev))
    x = feats.from_ids(tok.to(dev), E.to(dev), s)
    x2 = feats(E.to(dev)[tok.to(dev)], s)                    # the reference signature, same kernel
    assert torch.equal(x, x2)
    out = mem(h.to(dev), None, router_in=x).cpu()
    _, codes_gpu = mem.route_codes(x)
    # oracle
    p = oracle_params(mem)
    fsd = {k: v.detach().cpu() for k, v in feats.state_dict().items()}
    s_ref = torch.from_numpy(om.ssm_scan(a.numpy(), u.numpy())).float()
    assert om.rel_err(s.cpu().double(), s_ref.double()) < 1e-5
    x_ref = om.router_features(E[tok], fsd["start"], fsd["prev_norm.weight"], fsd["cur_norm.weight"], w.norm_eps,
                               s_ref)
    assert om.rel_err(x.cpu().double(), x_ref.double()) < 4e-3
    q64 = om.router_logits(x.cpu(), p["router.weight"]).numpy()   # codes of the GPU's own features
    codes, _ = codes_check(codes_gpu.cpu().numpy().astype(np.int32), q64)
    ref = om.memory_forward(p, cfg_of(w), h, codes)
    assert om.rel_err(out, ref) < 2e-2
    ref64 = om.memory_forward(p, cfg_of(w), h.double(), codes)
    assert om.rel_err(out, ref64) < 2e-2


def test_sdc_full_size_sampled(dev):
    """The full SD-C shape (8 x 4096 tokens, R181, 256-channel SSM): the scan and the router features
    against the oracle, every code against the fp64 router (outside the near-tie band), and the
    layer output at sampled positions against the bf16 and fp64 oracles of their 12-position
    causal windows (the conv's halo is 9 positions, the n-grams reach 2 back)."""
    from .test_gpu_memory import _window_oracle

    w = workloads.SDC
    mem, E, tok, a, u, h = _sdc_pipeline(w, dev, seed=3)
    feats = mem.router_features
    s = ops.ssm_scan(a.to(dev), u.to(dev))
    x = feats.from_ids(tok.to(dev), E.to(dev), s)
    out = mem(h.to(dev), None, router_in=x)
    assert out.shape == (8, 4096, 1024) and bool(torch.isfinite(out).all())
    _, codes_gpu = mem.route_codes(x)
    s_ref = torch.from_numpy(om.ssm_scan(a.numpy(), u.numpy()))
    assert om.rel_err(s.cpu().double(), s_ref) < 1e-5
    p = oracle_params(mem)
    fsd = {k: v.detach().cpu() for k, v in feats.state_dict().items()}
    for b in (0, 5):                                          # whole sequences of two batch rows
        want = om.router_features(E[tok[b]][None], fsd["start"], fsd["prev_norm.weight"], fsd["cur_norm.weight"],
                                  w.norm_eps, s.cpu()[b][None])
        assert om.rel_err(x[b].cpu().double(), want[0].double()) < 4e-3, b
    rng = np.random.default_rng(1)
    q64 = om.router_logits(x.reshape(-1, x.shape[-1]).cpu(), p["router.weight"]).numpy().reshape(8, 4096, -1)
    codes, near = codes_check(codes_gpu.cpu().numpy().astype(np.int32), q64)
    print(f"near-tie routes at SD-C size: {near} of {codes.size}")
    out_given = mem.module(h.to(dev), torch.as_tensor(codes, device=dev)).cpu()
    picks = [(0, 0), (0, 1), (0, 2), (4, 9), (7, 4095)] + [(int(rng.integers(0, 8)), int(rng.integers(0, 4096)))
                                                          for _ in range(11)]
    cfg = cfg_of(w)
    got = torch.stack([out_given[b, t] for b, t in picks])
    want = torch.stack([_window_oracle(p, cfg, h, codes, b, t) for b, t in picks])
    want64 = torch.stack([om.memory_forward(p, cfg, h[b:b + 1, max(0, t - 11):t + 1].double(),
                                            codes[b:b + 1, max(0, t - 11):t + 1])[0, -1] for b, t in picks])
    assert om.rel_err(got, want) < 2e-2
    assert om.rel_err(got, want64) < 2e-2


@pytest.mark.parametrize("which", ["sdc", "sdb"])
def test_router_codes_from_ids_equal_materialised_features(dev, which):
    """The router GEMM over rows gathered from the tabled embedding norms (lng_router_codes_ids) against
    the materialised features + router GEMM (lng_router_features + lng_router_codes, pinned to the
    oracle above): the tables equal the features' halves, and codes, logits and the layer output are
    bit-identical, with ids outside the vocabulary and sequence starts in the batch."""
    base = workloads.SDC if which == "sdc" else workloads.SDB
    w = base.with_shape(2, 2048)                              # 4096 tokens: the gathered GEMM's smallest M
    mem, E, tok, a, u, h = _sdc_pipeline(w, dev, seed=5)
    V, d = w.vocab, w.d_model
    tok[0, 7] = -1
    tok[1, 100] = V
    tok[1, 5] = V + 9
    E, tok, h = E.to(dev), tok.to(dev), h.to(dev)
    feats = mem.router_features
    s = sb = None
    if which == "sdc":
        s, sb = ops.ssm_scan(a.to(dev), u.to(dev), want_bf16=True)
        assert torch.equal(s, ops.ssm_scan(a.to(dev), u.to(dev)))
        assert torch.equal(sb, s.to(torch.bfloat16))
    x = feats.from_ids(tok, E, s)
    fprev, fcur = feats.tables(E)
    assert fprev.shape == (V + 2, d) and fcur.shape == (V + 1, d)
    valid = (tok >= 0) & (tok < V)
    idc = torch.where(valid, tok, V)
    idp = torch.cat((torch.full_like(idc[:, :1], V), torch.where(valid, tok, V + 1)[:, :-1]), 1)
    assert torch.equal(x[..., :d], fprev[idp]) and torch.equal(x[..., d:2 * d], fcur[idc])
    assert not bool(fprev[V + 1].any()) and not bool(fcur[V].any())
    n = 0 if sb is None else sb.shape[-1]
    assert ops.router_codes_ids_ok(tok.numel(), d, n, mem.router.weight.shape[0])
    lg_ref, codes_ref = mem.route_codes(x, want_logits=True)
    lg, codes = ops.router_codes_ids(tok, fprev, fcur, sb, mem.router.weight, want_logits=True)
    assert torch.equal(codes, codes_ref) and torch.equal(lg, lg_ref)
    with torch.no_grad():
        out_ref = mem(h, None, router_in=x)
        out = mem.forward_ids(h, tok, E, sb)
        out32 = mem.forward_ids(h, tok, E, s)                 # fp32 states are rounded the same way
    assert torch.equal(out, out_ref) and torch.equal(out32, out_ref)
