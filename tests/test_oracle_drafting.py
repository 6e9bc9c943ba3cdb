"""Pins of the drafting oracle (CPU): the reference's own known answers for the tree helpers and
acceptance (``tests/test_live_tree.py:17-52``), the drafter invariants its tests hold
(``tests/test_live_drafter.py:22-73``: draft = teacher-forced chain, no mutation, exact
rollback, commit in pieces), the online-counts repeated-pattern rule
(``tests/test_drafting_drafters.py:151-160``), closed forms (zero tables), and the draft head
against an independent restatement in the module form of ``DraftReadout.hidden``
(``ffnmem/memory/draft.py:73-86``)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from lngram_hip import workloads as wl
from oracle import drafting as od
from oracle import memory as om

PARENT = (-1, 0, 1, 0, 3, 1)  # 0 -> {1, 3}; 1 -> {2, 5}; 3 -> {4}


# ----------------------------------------------------------------------------- tree known answers
def test_mask_and_ancestor_codes_known_answers():
    m = od.tree_attention_mask(PARENT, 2)
    expect = np.array([[1, 1, 1, 0, 0, 0, 0, 0],
                       [1, 1, 1, 1, 0, 0, 0, 0],
                       [1, 1, 1, 1, 1, 0, 0, 0],
                       [1, 1, 1, 0, 0, 1, 0, 0],
                       [1, 1, 1, 0, 0, 1, 1, 0],
                       [1, 1, 1, 1, 0, 0, 0, 1]], dtype=bool)
    assert np.array_equal(m, expect)
    assert (5 + np.array(od.tree_depths(PARENT))).tolist() == [5, 6, 7, 6, 7, 7]
    codes = np.array([0, 10, 20, 30, 40, 50]).reshape(1, 6, 1)
    hist = np.array([100, 101]).reshape(1, 2, 1)
    ctx, ok = od.tree_ngram_codes(PARENT, codes, hist, 2)
    assert ctx[0, :, :, 0].tolist() == [[100, 101, 0], [101, 0, 10], [0, 10, 20], [101, 0, 30], [0, 30, 40],
                                        [0, 10, 50]]
    assert ok.all()
    ctx, ok = od.tree_ngram_codes(PARENT, codes, None, 2)
    assert ok.tolist() == [[False, False, True], [False, True, True], [True, True, True], [False, True, True],
                           [True, True, True], [True, True, True]]
    assert ctx[0, 1, :, 0].tolist() == [0, 0, 10] and ctx[0, 4, :, 0].tolist() == [0, 30, 40]
    with pytest.raises(ValueError):
        od.TreeSpec((-1, 2, 0), (0, 0, 0))


def test_tree_accept_known_answers():
    toks = [7, 1, 2, 3, 4, 5]
    assert od.tree_accept(PARENT, toks, [3, 9, 9, 4, 8, 9]) == ([0, 3, 4], [3, 4, 8])
    assert od.tree_accept(PARENT, toks, [1, 5, 9, 9, 9, 6]) == ([0, 1, 5], [1, 5, 6])
    assert od.tree_accept(PARENT, toks, [9, 9, 9, 9, 9, 9]) == ([0], [9])


def test_sixteen_node_tree_is_valid_and_has_ten_parents_in_four_depths():
    spec = od.TreeSpec((-1, 0, 1, 2, 3, 0, 5, 6, 7, 1, 9, 10, 2, 12, 3, 0),
                       (0, 0, 0, 0, 0, 1, 0, 0, 0, 1, 0, 0, 1, 0, 1, 2))
    parents = sorted(set(spec.parent[1:]))
    assert len(parents) == 10
    depth = od.tree_depths(spec.parent)
    assert sorted({depth[p] for p in parents}) == [0, 1, 2, 3]


def test_tree_route_tokens_equal_chain_lookup_of_each_path():
    # the verify gather of node i equals the route tokens at the end of its root->i path decoded
    # as a plain sequence (history + path), so tree order never leaks into a node's window
    rng = np.random.default_rng(3)
    r, bits, md = 3, 4, 4
    tables = {n: torch.randn(r * 16 ** n, md, dtype=torch.float64) for n in (2, 3)}
    hist = rng.integers(0, 16, (1, 5, r))
    codes = rng.integers(0, 16, (1, len(PARENT), r))
    ctx, ok = od.tree_ngram_codes(PARENT, codes, hist, 2)
    got = od.tree_route_tokens(tables, (2, 3), bits, ctx, ok)
    for i in range(len(PARENT)):
        path = od.tree_path(PARENT, i)
        seq = np.concatenate((hist[0], codes[0, path]), 0)[None]
        want = om.route_tokens(tables, seq, (2, 3), bits)[0, -1]
        torch.testing.assert_close(got[0, i], want)
    # no history: n-grams reaching before the root are zero
    ctx, ok = od.tree_ngram_codes(PARENT, codes, None, 2)
    got = od.tree_route_tokens(tables, (2, 3), bits, ctx, ok)
    assert float(got[0, 0].abs().sum()) == 0.0                      # root: no complete n-gram
    assert float(got[0, 1, :, md:].abs().sum()) == 0.0              # depth 1: no 3-gram


# ----------------------------------------------------------------------------- drafter invariants
@pytest.fixture(scope="module", params=["sdb", "sdc"])
def bundle(request):
    w = wl.TINY_DRAFT if request.param == "sdb" else wl.TINY_DRAFT_SSM
    cfg, t = wl.build_draft_bundle(w, seed=5)
    g = torch.Generator().manual_seed(9)
    for k in ("router_prev_norm", "router_cur_norm", "q_norm", "out_norm", "mem_norm"):  # exercise the weights
        t[k] = (1 + 0.2 * torch.randn(t[k].shape, generator=g)).to(t[k].dtype)
    return cfg, t


def chain_by_trace(cfg, t, prefix, gamma) -> list:
    seq, out = list(prefix), []
    for _ in range(gamma):
        _, lg = od.DrafterOracle(cfg, t).trace(seq)
        nxt = int(od.top_order(torch.from_numpy(lg[-1]), 1)[0])
        out.append(nxt)
        seq.append(nxt)
    return out


def test_draft_equals_teacher_forced_chain(bundle):
    cfg, t = bundle
    d = od.DrafterOracle(cfg, t)
    prefix = torch.randint(0, cfg["vocab"], (20,), generator=torch.Generator().manual_seed(1)).tolist()
    d.commit(prefix)
    out = d.draft(4)
    assert out.tokens == chain_by_trace(cfg, t, prefix, 4)
    assert out.topk_ids.shape == (4, 3) and (out.topk_ids[:, 0] == out.tokens).all()
    assert (np.diff(out.topk_logits, axis=1) <= 0).all()
    assert out.codes.shape == (3, cfg["routes"])
    assert d.draft(4, last_codes=True).codes.shape == (4, cfg["routes"])


def test_draft_does_not_mutate_and_rollback_is_exact(bundle):
    cfg, t = bundle
    g = torch.Generator().manual_seed(2)
    a = torch.randint(0, cfg["vocab"], (15,), generator=g).tolist()
    b = torch.randint(0, cfg["vocab"], (7,), generator=g).tolist()
    d = od.DrafterOracle(cfg, t)
    d.commit(a)
    first = d.draft(3)
    codes_a = d.committed_codes().copy()
    d.draft(5, hyp=b)
    assert d.length == 15 and d.draft(3).tokens == first.tokens
    d.commit(b)
    with_b = d.draft(3)
    d.truncate(15)
    np.testing.assert_array_equal(d.committed_codes(), codes_a)
    assert d.draft(3).tokens == first.tokens
    assert d.draft(3, hyp=b).tokens == with_b.tokens
    e = od.DrafterOracle(cfg, t)
    for i in range(0, 15, 4):
        e.commit(a[i:i + 4])
    np.testing.assert_array_equal(e.committed_codes(), codes_a)
    d.reset()
    with pytest.raises(ValueError):
        d.draft(1)


def test_chain_tree_equals_chain_draft(bundle):
    cfg, t = bundle
    d = od.DrafterOracle(cfg, t)
    d.commit(torch.randint(0, cfg["vocab"], (12,), generator=torch.Generator().manual_seed(4)).tolist())
    gamma = 3
    toks = od.draft_tree(d, od.TreeSpec((-1,) + tuple(range(gamma)), (0,) * (gamma + 1)))
    assert toks[0] == d.tokens[-1] and toks[1:] == d.draft(gamma).tokens


def test_zero_tables_give_zero_hidden_and_tie_order(bundle):
    # all route tokens zero -> scores 0 -> zero values -> W_o 0 = 0 -> RMSNorm(0) = 0 -> every logit 0:
    # top-k is then decided by the tie rule alone (index ascending)
    cfg, t = bundle
    t0 = dict(t)
    for n in cfg["ngrams"]:
        t0[f"table_{n}"] = torch.zeros_like(t[f"table_{n}"])
    t0.pop("w_sq", None)
    d = od.DrafterOracle(cfg, t0)
    d.commit([5, 6, 7, 8])
    cur = d._cursor()
    assert float(d.hidden(cur).abs().max()) == 0.0
    assert d.draft(1, topk=4).topk_ids[0].tolist() == [0, 1, 2, 3]


def test_draft_head_matches_module_form_restatement(bundle):
    # DraftReadout.hidden (draft.py:73-86) in the memory module's own ops: _project_memory
    # (memory norm + kv projection), scores via matmul, _real_route_probabilities, W_o, out_norm
    cfg, t = bundle
    d = od.DrafterOracle(cfg, t)
    d.commit(torch.randint(0, cfg["vocab"], (9,), generator=torch.Generator().manual_seed(6)).tolist())
    cur = d._cursor()
    rows = d.rows(cur)
    f64 = {k: v.double() for k, v in t.items() if v.is_floating_point()}
    tok = torch.cat([f64[f"table_{n}"][torch.from_numpy(rows[n])] for n in cfg["ngrams"]], -1)
    mc = om.MemCfg(cfg["d_model"], cfg["routes"], cfg["mem_dim"], cfg["q_heads"], cfg["kv_heads"], cfg["head_dim"],
                   eps=cfg["mem_eps"])
    params = {"readout_memory_norm.weight": f64["mem_norm"], "readout_kv_proj.weight": f64["kv_proj"]}
    key, value = om.project_memory(params, mc, tok[None, None])     # [1, 1, kv, R, hd]
    e = f64["embedding"][cur.tok]
    q = om.rms_norm(e, f64["q_norm"], cfg["draft_eps"]) @ f64["w_q"].T
    if "w_sq" in f64:
        q = q + f64["w_sq"] @ cur.s
    q = q.view(cfg["kv_heads"], cfg["groups"], cfg["head_dim"])
    scores = torch.matmul(q, key[0, 0].transpose(-1, -2)) * cfg["softmax_scale"]
    probs = om.sink_probabilities(scores, cfg["sink_logit"])
    out = torch.matmul(probs, value[0, 0]).reshape(-1)
    want = om.rms_norm(f64["w_o"] @ out, f64["out_norm"], cfg["draft_eps"])
    torch.testing.assert_close(d.hidden(cur), want, rtol=1e-10, atol=1e-12)


def test_fp32_restatement_close_to_fp64(bundle):
    cfg, t = bundle
    toks = torch.randint(0, cfg["vocab"], (30,), generator=torch.Generator().manual_seed(7)).tolist()
    c64, l64 = od.DrafterOracle(cfg, t).trace(toks)
    c32, l32 = od.DrafterOracle(cfg, t, dtype=torch.float32).trace(toks, codes=c64)
    assert np.abs(l32 - l64).max() < 1e-4 * max(1.0, np.abs(l64).max())


# ----------------------------------------------------------------------------- online counts
def test_online_counts_continue_a_repeated_pattern(bundle):
    # drafters.py:117-142 with a zero base distribution: the counts alone continue the pattern once
    # its windows repeat (every full row accepts; tests/test_drafting_drafters.py:151-160)
    cfg, t = bundle
    if "w_sq" in t:
        pytest.skip("codes depend on the SSM state, which does not repeat with the pattern")
    pat = [7, 30, 41, 52, 63]
    toks = pat * 8
    d = od.DrafterOracle(cfg, t)
    d.commit(toks)
    codes = d.committed_codes()
    n = len(toks)
    hits = 0
    for last in range(12, n - 1):
        win = codes[last - 2: last + 1][None]
        real = np.ones((1, 3), bool)
        p0 = torch.zeros(1, cfg["vocab"], dtype=torch.float64)
        p = od.online_counts_mix(p0, codes, toks, cfg["ngrams"], cfg["bits"], win, real, [last - 1])
        hits += int(int(p.argmax()) == toks[last + 1])
    assert hits == n - 1 - 12


def test_online_mix_closed_forms(bundle):
    cfg, t = bundle
    rng = np.random.default_rng(0)
    v = cfg["vocab"]
    codes = rng.integers(0, 16, (40, cfg["routes"]))
    x = rng.integers(0, v, 40)
    p = torch.softmax(torch.randn(2, v, dtype=torch.float64), -1)
    win = codes[[[17, 18, 19], [30, 31, 32]]]
    real = np.ones((2, 3), bool)
    # nothing verified yet: the distribution is unchanged
    torch.testing.assert_close(od.online_counts_mix(p, codes, x, (2, 3), 4, win, real, [-1, -1]), p)
    q = od.online_counts_mix(p, codes, x, (2, 3), 4, win, real, [38, 38])
    torch.testing.assert_close(q.sum(-1), torch.ones(2, dtype=torch.float64))
    # a window equal to an earlier pair's window: that pair's next token gains mass
    assert (q[:, x[1:]].sum(-1) >= p[:, x[1:]].sum(-1) - 1e-12).all()
