"""The product's module mirrors on the GPU against the oracle (``-m gpu``):

- ``lookup_rows_at`` (``draft.py:26-47``): equal to the full lookup at the sampled positions,
  windows that cross position 0 included;
- ``DraftReadout.hidden / forward`` (``draft.py:73-91``) in fp32 within 1e-5 of the fp64 oracle
  composition (memory projection, grouped sink attention, ``W_o``, RMSNorm), with and without
  the SSM query term;
- ``drafting.tree`` ``tree_ngram_codes`` / ``tree_route_tokens`` (``tree.py:114-136``) bit-exact;
- ``drafting.drafters`` ``window_rows`` and ``OnlineCounts.mix`` (``drafters.py:99-142``);
- ``LngramMemory.diagnostics`` (``wrapper.py:174-220``): code histogram statistics and sink mass;
- ``DiagonalSSM.forward / step`` and ``TokenRouterFeatures.step`` (``ssm.py:37-55``,
  ``router.py:61-68``);
- ``lng_ngram_rows`` with int64 rows past the int32 range, and its refusal of int32 there;
- ``make_drafter`` for every ``impl`` of the reference, and ``draft`` on a worker thread while the
  main thread launches kernels (``live_spec.py:316-319``).
"""

from __future__ import annotations

import threading
from dataclasses import replace

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from drafting import drafters as ddr
from drafting import tree as dtree
from drafting.cpu_drafter import make_drafter
from drafting.gpu_drafter import GpuDrafter
from ffnmem.memory import draft as mdraft
from ffnmem.memory import router as mrouter
from ffnmem.memory import ssm as mssm
from lngram_hip import ops, workloads
from oracle import drafting as od
from oracle import memory as om

pytestmark = pytest.mark.gpu


def _tiny_memory(dev):
    w = workloads.TINY
    mem = workloads.build_memory(w, seed=0, device=dev)
    cfg = om.MemCfg(w.d_model, w.routes, w.mem_dim, w.q_heads, w.kv_heads, w.head_dim, eps=w.norm_eps)
    sd = {k: v.detach().cpu() for k, v in mem.state_dict().items()}
    p = {k[len("module."):]: v for k, v in sd.items() if k.startswith("module.")}
    p["router.weight"] = sd["router.weight"]
    return mem, cfg, p


def _codes(shape, seed, dev):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 16, shape, generator=g, dtype=torch.int32).to(dev)


def test_lookup_rows_at_equals_full_lookup(dev):
    mem, cfg, p = _tiny_memory(dev)
    m = mem.module
    codes = _codes((3, 20, cfg.routes), 1, dev)
    b_idx = torch.tensor([0, 0, 1, 2, 2, 1, 0], device=dev)
    t_idx = torch.tensor([0, 1, 2, 19, 5, 0, 13], device=dev)
    got = mdraft.lookup_rows_at(m, codes, None, b_idx, t_idx).cpu()
    tables = {n: p[f"tables.ngram_{n}.weight"] for n in cfg.orders}
    full = om.route_tokens(tables, codes.cpu().numpy(), cfg.orders, cfg.bits)
    want = full[b_idx.cpu(), t_idx.cpu()]
    assert torch.equal(got, want)


@pytest.mark.parametrize("ssm_dim", [0, 8])
def test_draft_readout_matches_oracle(dev, ssm_dim):
    mem, cfg, p = _tiny_memory(dev)
    m = mem.module
    torch.manual_seed(3)
    dr = mdraft.DraftReadout(cfg.d_model, m, q_heads=4, head_dim=cfg.head_dim, ssm_dim=ssm_dim).to(dev)
    with torch.no_grad():
        dr.q_norm.weight.copy_(1 + 0.1 * torch.randn(cfg.d_model))
        dr.out_norm.weight.copy_(1 + 0.1 * torch.randn(cfg.d_model))
    n, vocab = 9, 77
    codes = _codes((2, 12, cfg.routes), 4, dev)
    b_idx, t_idx = torch.tensor([0, 1, 1, 0, 1, 0, 0, 1, 1], device=dev), torch.arange(9, device=dev) + 2
    rt = mdraft.lookup_rows_at(m, codes, None, b_idx, t_idx)
    emb = torch.randn(n, cfg.d_model, device=dev)
    unembed = torch.randn(vocab, cfg.d_model, device=dev)
    s = torch.randn(n, ssm_dim, device=dev) if ssm_dim else None
    got_h = dr.hidden(m, emb, rt, s).cpu()
    got = dr.forward(m, emb, rt, unembed, s).cpu()
    # oracle composition in fp64
    d64 = {k: v.detach().cpu().double() for k, v in dr.state_dict().items()}
    key, value = om.project_memory({k: v.double() for k, v in p.items()}, cfg, rt.cpu().double()[:, None])
    q = F.linear(om.rms_norm(emb.cpu().double(), d64["q_norm.weight"], cfg.eps), d64["w_q.weight"])
    if ssm_dim:
        q = q + F.linear(s.cpu().double(), d64["w_sq.weight"])
    dcfg = replace(cfg, q_heads=4)
    o = om.manual_gqa(dcfg, q.view(n, 1, 4, cfg.head_dim), key, value).reshape(n, -1)
    h = om.rms_norm(F.linear(o, d64["w_o.weight"]), d64["out_norm.weight"], cfg.eps)
    assert om.rel_err(got_h, h) < 1e-5
    assert om.rel_err(got, h @ unembed.cpu().double().T) < 1e-5


@pytest.mark.parametrize("spec", [dtree.tree16(), dtree.default_tree(), dtree.chain_tree(4)])
def test_tree_windows_and_route_tokens_match_oracle(dev, spec):
    mem, cfg, p = _tiny_memory(dev)
    m = mem.module
    n = spec.n
    node_codes = _codes((2, n, cfg.routes), 5, dev)
    for hist in (None, _codes((2, 3, cfg.routes), 6, dev)):
        ctx, ok = dtree.tree_ngram_codes(spec.parent, node_codes, hist, 2)
        wctx, wok = od.tree_ngram_codes(spec.parent, node_codes.cpu().numpy(),
                                        None if hist is None else hist.cpu().numpy(), 2)
        assert (ctx.cpu().numpy() == wctx).all() and (ok.cpu().numpy() == wok).all()
        got = dtree.tree_route_tokens(m, ctx, ok).cpu()
        tables = {k: p[f"tables.ngram_{k}.weight"] for k in cfg.orders}
        want = od.tree_route_tokens(tables, cfg.orders, cfg.bits, wctx, wok)
        assert torch.equal(got, want)


def test_window_rows_and_online_counts_match_oracle(dev):
    g = torch.Generator().manual_seed(7)
    t_len, r, vocab, n = 60, 5, 40, 12
    pat = torch.randint(0, 16, (5, r), generator=g)
    codes = torch.cat([pat] * 8 + [torch.randint(0, 16, (t_len - 40, r), generator=g)])  # repeats -> matches
    x = torch.randint(0, vocab, (t_len,), generator=g)
    win = torch.randint(0, 16, (n, 3, r), generator=g)
    win[:6] = codes[torch.arange(6)[:, None] + torch.arange(3)[None] + 10]     # windows of committed positions
    real = torch.ones(n, 3, dtype=torch.bool)
    real[7, :2] = False
    real[8, :1] = False
    deadline = torch.randint(0, t_len - 1, (n,), generator=g)
    p = torch.softmax(torch.randn(n, vocab, generator=g, dtype=torch.float64), -1)
    for order in (2, 3):
        got = ddr.window_rows(win.to(dev), real.to(dev), order, 4).cpu().numpy()
        assert (got == od.window_rows(win.numpy(), real.numpy(), order, 4)).all()
    oc = ddr.OnlineCounts(codes.to(dev), x.to(dev), (2, 3), 4, vocab)
    got = oc.mix(p.float().to(dev), win.to(dev), real.to(dev), deadline.to(dev)).cpu().double()
    want = od.online_counts_mix(p, codes.numpy(), x.numpy(), (2, 3), 4, win.numpy(), real.numpy(),
                                deadline.numpy())
    assert (want != p).any()                       # some rows matched pairs
    assert om.rel_err(got, want) < 1e-5
    assert torch.equal(got.argmax(-1), want.argmax(-1))


def test_diagnostics_match_oracle(dev):
    mem, cfg, p = _tiny_memory(dev)
    w = workloads.TINY
    mem.eval()
    mem.collect_diagnostics = True
    h = workloads.make_hidden(w, seed=8, device=dev)
    h_norm = ops.rmsnorm(h, torch.ones(w.d_model, device=dev), w.norm_eps)
    mem(h, h_norm)
    got = mem.diagnostics()
    _, codes = mem.route_codes(h_norm)
    c = codes.cpu().numpy().astype(np.int64).reshape(-1, cfg.routes)
    hist = np.stack([np.bincount(c[:, r], minlength=16) for r in range(cfg.routes)]).astype(np.float64)
    pr = hist / hist.sum(-1, keepdims=True)
    eff = np.exp(-(pr * np.log(np.clip(pr, 1e-30, None))).sum(-1))
    assert abs(got["eff_codes_mean"] - eff.mean()) < 1e-9
    assert abs(got["dead_code_frac"] - (hist == 0).mean()) < 1e-12
    assert abs(got["top_code_share"] - pr.max(-1).mean()) < 1e-9
    assert abs(got["frac_routes_eff_lt4"] - (eff < 4).mean()) < 1e-12
    # sink mass: 1 - sum of the real-route probabilities (fp64 oracle scores)
    q = om.project_query({k: v.double() for k, v in p.items()}, cfg, h.cpu().double())
    tok = om.route_tokens({n: p[f"tables.ngram_{n}.weight"].double() for n in cfg.orders}, c.reshape(*h.shape[:2], -1),
                          cfg.orders, cfg.bits)
    key, _ = om.project_memory({k: v.double() for k, v in p.items()}, cfg, tok)
    grouped = q.view(*h.shape[:2], cfg.kv_heads, cfg.groups, cfg.head_dim)
    scores = torch.matmul(grouped, key.transpose(-1, -2)) * cfg.softmax_scale
    sink = 1 - om.sink_probabilities(scores, cfg.sink_logit).sum(-1)
    assert abs(got["sink_mass"] - float(sink.mean())) < 1e-5


def test_ssm_forward_step_and_router_step(dev):
    torch.manual_seed(9)
    s = mssm.DiagonalSSM(48, 16, chunk=8).to(dev)
    with torch.no_grad():
        s.norm.weight.copy_(1 + 0.1 * torch.randn(48))
    emb = torch.randn(2, 21, 48, device=dev)
    got = s(emb).cpu()
    u = om.ssm_inputs(emb.cpu(), s.norm.weight.detach().cpu(), s.w_in.weight.detach().cpu(), s.norm.eps)
    want = om.ssm_scan(s.decay().detach().cpu().numpy(), u.numpy())
    assert om.rel_err(got, want) < 1e-5
    st = None
    for i in range(4):
        st = s.step(st, emb[:, i])
    assert om.rel_err(st.cpu(), want[:, 3]) < 1e-5
    for kind in ("embed2", "embed2_ssm"):
        f = mrouter.TokenRouterFeatures(64, kind).to(dev)
        with torch.no_grad():
            f.prev_norm.weight.copy_(1 + 0.1 * torch.randn(64))
        e = torch.randn(3, 5, 64, device=dev)
        ss = torch.randn(3, 5, 16, device=dev) if kind == "embed2_ssm" else None
        seq = f(e, ss)
        for t in (0, 3):
            one = f.step(None if t == 0 else e[:, t - 1], e[:, t], None if ss is None else ss[:, t])
            assert torch.equal(one, seq[:, t])


def test_ngram_rows_int64_past_int32(dev):
    # bits 8, order 3, 130 routes: the largest row is 130 * 2^24 - 1 > 2^31 - 1
    g = torch.Generator().manual_seed(10)
    codes = torch.randint(0, 256, (2, 7, 130), generator=g, dtype=torch.int32)
    got = ops.ngram_rows(codes.to(dev), (2, 3), 8).cpu()
    assert got.dtype == torch.int64
    assert (got.numpy() == om.route_rows(codes.numpy(), (2, 3), 8)).all()
    assert int(got.max()) > 2 ** 31
    with pytest.raises(RuntimeError, match="int32"):
        ops.ngram_rows(codes.to(dev), (2, 3), 8, rows_dtype=torch.int32)


def test_make_drafter_impls_and_worker_thread_draft(dev):
    cfg, t = workloads.build_draft_bundle(workloads.TINY_DRAFT, seed=5)
    toks = torch.randint(0, cfg["vocab"], (40,), generator=torch.Generator().manual_seed(11)).tolist()
    ds = [make_drafter((cfg, t), impl, threads=2, device=dev, max_len=64) for impl in ("ref", "cpp", "auto", "gpu")]
    assert all(isinstance(d, GpuDrafter) for d in ds)
    with pytest.raises(ValueError):
        make_drafter((cfg, t), "bogus")
    d = ds[0]
    d.commit(toks)
    want = d.draft(5, toks[-3:], None, True)
    # live_spec submits draft(gamma + 1, D, None, need_codes) to a worker while the main thread verifies
    out: dict = {}

    def worker():
        out["d"] = d.draft(5, toks[-3:], None, True)

    th = threading.Thread(target=worker)
    th.start()
    x = torch.randn(512, 512, device=dev)
    for _ in range(20):
        x = ops.linear(x, x).clamp(-1, 1)       # the verifier's work on the main thread's stream
    th.join()
    torch.cuda.synchronize()
    got = out["d"]
    assert got.tokens == want.tokens and (got.topk_ids == want.topk_ids).all() and (got.codes == want.codes).all()
    assert d.length == len(toks)
