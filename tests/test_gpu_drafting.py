"""Parity of the GPU drafter (``drafting.gpu_drafter.GpuDrafter``) with the drafting oracle (GPU).

Route codes are compared bit-exactly outside the near-tie band |router logit| < 2e-5 (the oracle's
fp64 logits decide which entries are ties); readouts are compared with identical committed codes
(``commit(tokens, codes=...)``), so a tie cannot leak into the windows.  Logits (fp32 on the GPU)
against the fp64 oracle: norm-relative error < 1e-5, and no entry further than 1e-5 of the largest
logit magnitude from it; draft tokens, top-k ids and tree node tokens: equal.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from drafting import tree as dtree
from drafting.gpu_drafter import GpuDrafter
from lngram_hip import workloads as wl
from oracle import drafting as od

pytestmark = pytest.mark.gpu

TAU = 2e-5
SPEC16 = dtree.tree16()


KINDS = ["sdb", "sdb_generic", "sdc", "sdb_fast"]


def _bundle(kind: str, seed: int = 5):
    w = {"sdb": wl.TINY_DRAFT, "sdb_generic": wl.TINY_DRAFT, "sdc": wl.TINY_DRAFT_SSM,
         "sdb_fast": wl.TINY_DRAFT_FAST}[kind]
    cfg, t = wl.build_draft_bundle(w, seed=seed)
    g = torch.Generator().manual_seed(9)
    for k in ("router_prev_norm", "router_cur_norm", "q_norm", "out_norm", "mem_norm"):
        t[k] = (1 + 0.2 * torch.randn(t[k].shape, generator=g)).to(t[k].dtype)
    return cfg, t


def _assert_logits(got: np.ndarray, want: np.ndarray, rel: float = 1e-5) -> None:
    """fp32 logits against fp64: same finite entries, norm-relative and scaled max-abs bounds."""
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    ok = np.isfinite(want)
    assert (np.isfinite(got) == ok).all()
    d, w = got[ok] - want[ok], want[ok]
    assert np.linalg.norm(d) <= rel * np.linalg.norm(w), np.linalg.norm(d) / np.linalg.norm(w)
    assert np.abs(d).max() <= rel * np.abs(w).max(), np.abs(d).max() / np.abs(w).max()


def _gpu(kind, cfg, t, dev, **kw) -> GpuDrafter:
    """sdb / sdb_fast: per-token tables (two launches per readout; sdb_fast has Dt = 64);
    sdb_generic / sdc: the general kernels.  At these tiny shapes trees take the per-depth
    readouts (the one-launch tree serves the SD drafters' shape)."""
    g = GpuDrafter((cfg, t), device=dev, tables=kind in ("sdb", "sdb_fast"), **kw)
    assert (g.luts is not None) == (kind in ("sdb", "sdb_fast"))
    return g


def _oracle_codes_and_ties(o: od.DrafterOracle, toks: list):
    """Oracle codes of a committed sequence and a mask [T, R] of routes with a near-tie bit."""
    o.reset()
    ties = []
    cur = o._cursor()
    for tok in toks:
        s = None
        if o.has_ssm:
            e = o.E[tok]
            u = o.ssm_w_in @ od._rms(e, o.ssm_norm, o.cfg["ssm_eps"])
            s = o.ssm_a * (cur.s if cur.s is not None else torch.zeros_like(u)) + (1 - o.ssm_a) * u
        lg = o.router_logits(cur.tok if cur.t >= 0 else -1, tok, s)
        ties.append((lg.abs() < TAU).view(o.R, o.bits).any(-1).numpy())
        cur = o._advance(cur, tok)
    o.commit(toks)
    return o.committed_codes(), np.stack(ties)


@pytest.mark.parametrize("kind", KINDS)
def test_commit_codes_match_oracle(dev, kind):
    cfg, t = _bundle(kind)
    toks = torch.randint(0, cfg["vocab"], (70,), generator=torch.Generator().manual_seed(1)).tolist()
    o = od.DrafterOracle(cfg, t)
    want, ties = _oracle_codes_and_ties(o, toks)
    g = _gpu(kind, cfg, t, dev, max_len=128)
    g.commit(toks[:33])
    g.commit(toks[33:])                      # in two pieces: the second continues the first
    got = g.committed_codes()
    assert got.shape == want.shape
    assert (got[~ties] == want[~ties]).all()
    if kind == "sdc":                         # SSM states follow the recurrence
        s_want = torch.stack(o._ssm).numpy()
        s_got = g.ssm_d[:len(toks), :g.N].cpu().numpy()
        np.testing.assert_allclose(s_got, s_want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("kind", KINDS)
def test_trace_logits_match_oracle(dev, kind):
    cfg, t = _bundle(kind)
    toks = torch.randint(0, cfg["vocab"], (37,), generator=torch.Generator().manual_seed(2)).tolist()
    o = od.DrafterOracle(cfg, t)
    codes, lg = o.trace(toks)
    g = _gpu(kind, cfg, t, dev, max_len=64)
    c_got, ids, l_got = g.trace(toks, codes=codes)
    np.testing.assert_array_equal(c_got, codes)
    assert ids.shape == (37, cfg["vocab"]) and (ids[0] == np.arange(cfg["vocab"])).all()
    _assert_logits(l_got, lg)
    assert (l_got.argmax(1) == lg.argmax(1)).all()
    assert g.length == 0                     # trace leaves the committed state alone


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("online", [False, True])
def test_draft_matches_oracle(dev, kind, online):
    cfg, t = _bundle(kind)
    gen = torch.Generator().manual_seed(3)
    pat = torch.randint(0, cfg["vocab"], (6,), generator=gen).tolist()
    toks = pat * 5 + torch.randint(0, cfg["vocab"], (11,), generator=gen).tolist() + pat[:3]
    o = od.DrafterOracle(cfg, t, online=online)
    codes, _ = _oracle_codes_and_ties(od.DrafterOracle(cfg, t), toks)
    o.reset()
    o.commit(toks, codes=codes)
    g = _gpu(kind, cfg, t, dev, max_len=96, online=online)
    g.commit(toks, codes=codes)
    for hyp, gamma, k, last in (((), 4, 3, False), (tuple(pat[3:5]), 3, 4, True), ((), 1, 1, False)):
        want = o.draft(gamma, hyp=hyp, topk=k, last_codes=last)
        got = g.draft(gamma, hyp=hyp, topk=k, last_codes=last)
        assert got.tokens == want.tokens, (hyp, gamma)
        np.testing.assert_array_equal(got.topk_ids, want.topk_ids)
        _assert_logits(got.topk_logits, want.topk_logits)
        np.testing.assert_array_equal(got.codes, want.codes)
    assert g.length == len(toks)
    # rollback: truncate then draft equals a drafter that never saw the tail
    g.truncate(20)
    o2 = od.DrafterOracle(cfg, t, online=online)
    o2.commit(toks[:20], codes=codes[:20])
    assert g.draft(3).tokens == o2.draft(3).tokens


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("online", [False, True])
def test_draft_tree_and_verify_gather_match_oracle(dev, kind, online):
    cfg, t = _bundle(kind)
    toks = torch.randint(0, cfg["vocab"], (50,), generator=torch.Generator().manual_seed(4)).tolist()
    codes, _ = _oracle_codes_and_ties(od.DrafterOracle(cfg, t), toks)
    o = od.DrafterOracle(cfg, t, online=online)
    o.commit(toks, codes=codes)
    g = _gpu(kind, cfg, t, dev, max_len=64, online=online)
    g.commit(toks, codes=codes)
    for spec in (SPEC16, dtree.default_tree(), dtree.chain_tree(5)):
        ospec = od.TreeSpec(spec.parent, spec.rank)
        want = od.draft_tree(o, ospec)
        assert g.draft_tree(spec) == want
        # node codes (drafter's router along each node's path) and the verification gather
        node_tok, rt = g.tree_step(spec, route_tokens=True)
        assert node_tok.cpu().tolist() == want
        node_codes = np.zeros((spec.n, cfg["routes"]), np.int64)
        node_codes[0] = codes[-1]
        for i in range(1, spec.n):
            path = od.tree_path(spec.parent, i)
            c = o.draft(1, hyp=[want[a] for a in path[1:]], last_codes=True).codes
            node_codes[i] = c[len(path) - 2]
        assert g.tree_error() == 0
        got_codes = g.codes_d[g.tree_row0 + 1: g.tree_row0 + spec.n].cpu().numpy()
        np.testing.assert_array_equal(got_codes, node_codes[1:])
        hist = codes[None, -3:-1].astype(np.int64)
        nodes = node_codes[None].copy()
        ctx, ok = od.tree_ngram_codes(spec.parent, nodes, hist, 2)
        tables = {n: t[f"table_{n}"] for n in cfg["ngrams"]}
        rt_want = od.tree_route_tokens(tables, cfg["ngrams"], cfg["bits"], ctx, ok)[0]
        torch.testing.assert_close(rt.cpu(), rt_want.to(rt.dtype), rtol=0, atol=0)


def test_tree_accept_on_device_known_answers(dev):
    parent = (-1, 0, 1, 0, 3, 1)
    toks = [7, 1, 2, 3, 4, 5]
    for am, path, new in (([3, 9, 9, 4, 8, 9], [0, 3, 4], [3, 4, 8]), ([1, 5, 9, 9, 9, 6], [0, 1, 5], [1, 5, 6]),
                          ([9] * 6, [0], [9])):
        assert dtree.tree_accept(parent, toks, torch.tensor(am, device=dev)) == (path, new)


def test_api_errors(dev):
    cfg, t = _bundle("sdb")
    g = GpuDrafter((cfg, t), device=dev, max_len=16)
    with pytest.raises(ValueError):
        g.draft(1)
    with pytest.raises(ValueError):
        g.commit([cfg["vocab"]])
    g.commit([1, 2, 3])
    with pytest.raises(ValueError):
        g.truncate(4)
    with pytest.raises(ValueError):
        g.commit([1, 2], codes=np.full((2, cfg["routes"]), 16))
    with pytest.raises(ValueError):
        g.commit(list(range(14)))
    assert g.length == 3


def test_sdb_shape_tree_step_matches_oracle(dev):
    # SD-B drafter shape: d 1024, V 32768, R 182, bf16 weights, 2048-token context, 16-node tree
    w = wl.SDB_DRAFT
    cfg, t = wl.build_draft_bundle(w, seed=0)
    ctx = wl.make_context(w, seed=0)
    o = od.DrafterOracle(cfg, t)
    g = GpuDrafter((cfg, t), device=dev, max_len=w.context + 8)
    g.commit(ctx)
    got = g.committed_codes()
    # the oracle's own codes for the last 64 positions (the windows the tree reads), with ties
    tail = 64
    o.commit(ctx[: -tail], codes=got[: -tail])
    cur = o._cursor()
    n_tie = n_bad = 0
    for i, tok in enumerate(ctx[-tail:]):
        lg = o.router_logits(cur.tok, tok, None)
        tie = (lg.abs() < TAU).view(o.R, o.bits).any(-1).numpy()
        cur = o._advance(cur, tok)
        want = cur.hist[-1]
        n_tie += int(tie.sum())
        n_bad += int((got[len(ctx) - tail + i] != want)[~tie].sum())
    assert n_bad == 0
    o.reset()
    o.commit(ctx, codes=got)
    spec = od.TreeSpec(SPEC16.parent, SPEC16.rank)
    want = od.draft_tree(o, spec)
    assert g.draft_tree(SPEC16) == want


def test_sdb_shape_one_launch_tree_matches_per_depth_launches_and_oracle(dev):
    """SD-B drafter shape with online counts: the one-launch tree (lng_drafter_tree_levels) equals
    the per-depth readouts (node tokens, node codes, verification gather, bit for bit) and the
    oracle: the oracle's draft tree, its router codes of every node outside the near-tie band, and
    its verification gather ``tree_route_tokens`` [16, 182, 256] (tree.py:96-136) of the nodes'
    windows, bit for bit."""
    w = wl.SDB_DRAFT
    cfg, t = wl.build_draft_bundle(w, seed=0)
    ctx = wl.make_context(w, seed=0)
    g1 = GpuDrafter((cfg, t), device=dev, max_len=w.context + 8, online=True)
    g0 = GpuDrafter((cfg, t), device=dev, max_len=w.context + 8, online=True, levels=False)
    assert g1.level_work is not None and g0.level_work is None
    g1.commit(ctx)
    committed = g1.committed_codes()
    g0.commit(ctx, codes=committed)
    o = od.DrafterOracle(cfg, t, online=True)
    o.commit(ctx, codes=committed)
    want = od.draft_tree(o, od.TreeSpec(SPEC16.parent, SPEC16.rank))
    rows = slice(g1.tree_row0, g1.tree_row0 + SPEC16.n)
    for rep in range(3):                                     # repeated calls reuse the workspace
        print(f"[sdb one-launch tree] call {rep}", flush=True)
        n1, r1 = g1.tree_step(SPEC16, route_tokens=True)
        n0, r0 = g0.tree_step(SPEC16, route_tokens=True)
        torch.cuda.synchronize()
        assert g1.tree_error() == 0
        assert g1._level_specs[(tuple(SPEC16.parent), tuple(SPEC16.rank))]
        assert n1.cpu().tolist() == n0.cpu().tolist() == want
        assert torch.equal(r1, r0)
        assert torch.equal(g1.codes_d[rows][1:], g0.codes_d[rows][1:])
    # node codes against the oracle's router (root = the last committed token)
    node_codes = g1.codes_d[rows].cpu().numpy().astype(np.int64)
    node_codes[0] = committed[-1]
    n_bad = 0
    for i in range(1, SPEC16.n):
        lg = o.router_logits(want[SPEC16.parent[i]], want[i], None)
        tie = (lg.abs() < TAU).view(o.R, o.bits).any(-1).numpy()
        bits = (lg > 0).view(o.R, o.bits).to(torch.int64).numpy()
        oc = (bits << np.arange(o.bits)).sum(-1)
        n_bad += int((node_codes[i] != oc)[~tie].sum())
    assert n_bad == 0
    # the verification gather against the oracle's, from the nodes' codes along their ancestors
    hist = committed[None, -3:-1].astype(np.int64)
    octx, ok = od.tree_ngram_codes(SPEC16.parent, node_codes[None], hist, 2)
    tables = {n: t[f"table_{n}"] for n in cfg["ngrams"]}
    rt_want = od.tree_route_tokens(tables, cfg["ngrams"], cfg["bits"], octx, ok)[0]
    assert tuple(rt_want.shape) == (16, 182, 256)
    assert torch.equal(r1.cpu(), rt_want.to(r1.dtype))
    # draft_tree reads the error word in its one copy and agrees
    assert g1.draft_tree(SPEC16) == want


def test_sdb_shape_graph_tree_step_replays_match_eager(dev):
    """The captured tree step (one HIP graph per tree shape) equals the eager launches on every
    replay, with eager drafter work (commits, truncations) between the replays."""
    w = wl.SDB_DRAFT
    cfg, t = wl.build_draft_bundle(w, seed=0)
    ctx = wl.make_context(w, seed=0)
    g = GpuDrafter((cfg, t), device=dev, max_len=w.context + 16, online=True)
    g.commit(ctx[:-6])
    extra = list(ctx[-6:])
    for rnd in range(4):
        node_e, rt_e = g.tree_step(SPEC16, route_tokens=True)
        node_e, rt_e = node_e.clone(), rt_e.clone()
        node_g, rt_g = g.tree_step(SPEC16, route_tokens=True, graph=True)
        torch.cuda.synchronize()
        assert torch.equal(node_g, node_e), rnd
        assert torch.equal(rt_g, rt_e), rnd
        # eager work between replays: the committed state moves on, and is rolled back once
        g.commit(extra[rnd: rnd + 1])
        if rnd == 2:
            g.truncate(g.length - 1)
            g.commit(extra[rnd: rnd + 1])
    node_e = g.tree_step(SPEC16, route_tokens=False)[0].clone()
    node_g = g.tree_step(SPEC16, route_tokens=False, graph=True)[0]
    torch.cuda.synchronize()
    assert torch.equal(node_g, node_e)


@pytest.mark.parametrize("online", [False, True])
def test_sdb_shape_launch_per_step_tree_matches_oracle(dev, online):
    """SD-B drafter shape, a context with repeated tokens: the one-launch tree (lng_drafter_tree_levels:
    selection by every block that needs a pick, vocabulary slices held across depths, device-coherent
    hand-offs) equals the oracle's draft tree over repeated steps with commits between them, for the
    16-node, default and chain trees (eager and graph-replayed), and the per-depth readouts of
    lng_drafter_tree bit for bit (node tokens, node codes, verification gather); the per-depth chain
    draft's top-k equals the oracle's."""
    w = wl.SDB_DRAFT
    cfg, t = wl.build_draft_bundle(w, seed=0)
    ctx = wl.make_context(w, seed=1)
    g1 = GpuDrafter((cfg, t), device=dev, max_len=w.context + 16, online=online)
    g0 = GpuDrafter((cfg, t), device=dev, max_len=w.context + 16, online=online, levels=False)
    assert g1.level_work is not None and g0.level_work is None
    g1.commit(ctx[:-8])
    g0.commit(ctx[:-8], codes=g1.committed_codes())
    o = od.DrafterOracle(cfg, t, online=online)
    o.commit(ctx[:-8], codes=g1.committed_codes())
    k = 0
    for spec in (SPEC16, dtree.default_tree(), dtree.chain_tree(5)):
        for rep in range(2):
            print(f"[sdb levels tree] online={online} n={spec.n} step {rep}", flush=True)
            n1, r1 = g1.tree_step(spec, route_tokens=True, graph=rep == 1)
            n1, r1 = n1.clone(), r1.clone()
            torch.cuda.synchronize()
            assert g1.tree_error() == 0
            assert g1._level_specs[(tuple(spec.parent), tuple(spec.rank))]
            assert n1.cpu().tolist() == od.draft_tree(o, od.TreeSpec(spec.parent, spec.rank))
            # the per-depth readouts, bit for bit (online counts included: the match window of the
            # first pair of each counting block once dropped its oldest code)
            n0, r0 = g0.tree_step(spec, route_tokens=True)
            torch.cuda.synchronize()
            assert n1.cpu().tolist() == n0.cpu().tolist()
            assert torch.equal(r1, r0)
            rows = slice(g1.tree_row0 + 1, g1.tree_row0 + spec.n)
            assert torch.equal(g1.codes_d[rows], g0.codes_d[rows])
            if rep == 0:
                d0, do = g0.draft(1, topk=4), o.draft(1, topk=4)
                assert d0.topk_ids.tolist() == do.topk_ids.tolist()
            nxt = ctx[-8 + k: -7 + k]
            g1.commit(nxt)
            g0.commit(nxt, codes=g1.committed_codes()[-1:])
            o.commit(nxt, codes=g1.committed_codes()[-1:])
            k += 1


def test_levels_tree_many_count_bearing_tokens_in_one_slice(dev):
    """Forty distinct next tokens of one vocabulary slice after the same three-token window, and a
    context that ends in that window: the slice's record carries more count-bearing tokens than its
    inline entries, so the one-launch tree's selection also reads the record's spill area.  Node
    tokens, node codes and the verification gather equal the per-depth readouts bit for bit, and the
    node tokens equal the oracle's draft tree (16-node and chain trees)."""
    w = wl.SDB_DRAFT
    cfg, t = wl.build_draft_bundle(w, seed=0)
    gen = torch.Generator().manual_seed(5)
    fill = torch.randint(4000, w.vocab, (256,), generator=gen).tolist()
    ctx = list(fill)
    for i in range(40):
        ctx += [1000, 2000, 3000, 10 + i]
    ctx += fill[:64] + [1000, 2000, 3000]
    g1 = GpuDrafter((cfg, t), device=dev, max_len=len(ctx) + 16, online=True)
    g0 = GpuDrafter((cfg, t), device=dev, max_len=len(ctx) + 16, online=True, levels=False)
    g1.commit(ctx)
    g0.commit(ctx, codes=g1.committed_codes())
    o = od.DrafterOracle(cfg, t, online=True)
    o.commit(ctx, codes=g1.committed_codes())
    for spec in (SPEC16, dtree.chain_tree(5)):
        print(f"[levels tree, many counts in one slice] n={spec.n}", flush=True)
        n1, r1 = g1.tree_step(spec, route_tokens=True)
        n1, r1 = n1.clone(), r1.clone()
        torch.cuda.synchronize()
        assert g1.tree_error() == 0
        assert g1._level_specs[(tuple(spec.parent), tuple(spec.rank))]
        n0, r0 = g0.tree_step(spec, route_tokens=True)
        torch.cuda.synchronize()
        assert n1.cpu().tolist() == n0.cpu().tolist()
        assert torch.equal(r1, r0)
        rows = slice(g1.tree_row0 + 1, g1.tree_row0 + spec.n)
        assert torch.equal(g1.codes_d[rows], g0.codes_d[rows])
        assert n1.cpu().tolist() == od.draft_tree(o, od.TreeSpec(spec.parent, spec.rank))


@pytest.mark.parametrize("n_ctx", [2048, 4200])
def test_levels_tree_pairs_past_the_key_cache_and_the_list(dev, n_ctx):
    """A context whose tokens all lie in the first vocabulary slice (160 tokens), so one block lists
    every committed pair: 2047 pairs pass the 48 whose match keys sit in LDS (the rest recompute
    their keys from the committed codes), and 4199 pairs pass the 4096-entry list (the pairs are
    then listed and counted per depth in rounds).  Node tokens, node codes and the verification
    gather equal the per-depth readouts bit for bit, and the node tokens equal the oracle's draft
    tree with online counts."""
    w = wl.SDB_DRAFT
    cfg, t = wl.build_draft_bundle(w, seed=0)
    gen = torch.Generator().manual_seed(n_ctx)
    ctx = torch.randint(0, 160, (n_ctx,), generator=gen).tolist()
    g1 = GpuDrafter((cfg, t), device=dev, max_len=n_ctx + 16, online=True)
    g0 = GpuDrafter((cfg, t), device=dev, max_len=n_ctx + 16, online=True, levels=False)
    assert g1.level_work is not None
    g1.commit(ctx)
    g0.commit(ctx, codes=g1.committed_codes())
    o = od.DrafterOracle(cfg, t, online=True)
    o.commit(ctx, codes=g1.committed_codes())
    for spec in (SPEC16, dtree.chain_tree(5)):
        print(f"[levels tree, {n_ctx - 1} pairs in one slice] n={spec.n}", flush=True)
        n1, r1 = g1.tree_step(spec, route_tokens=True)
        n1, r1 = n1.clone(), r1.clone()
        torch.cuda.synchronize()
        assert g1.tree_error() == 0
        assert g1._level_specs[(tuple(spec.parent), tuple(spec.rank))]
        n0, r0 = g0.tree_step(spec, route_tokens=True)
        torch.cuda.synchronize()
        assert n1.cpu().tolist() == n0.cpu().tolist()
        assert torch.equal(r1, r0)
        rows = slice(g1.tree_row0 + 1, g1.tree_row0 + spec.n)
        assert torch.equal(g1.codes_d[rows], g0.codes_d[rows])
        assert n1.cpu().tolist() == od.draft_tree(o, od.TreeSpec(spec.parent, spec.rank))
