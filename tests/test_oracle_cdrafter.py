"""The C++ CPU drafter port (``oracle/c/cpu_drafter.cpp``, the drafter CPU baseline) against the
drafting oracle (CPU): codes bit-exact outside the near-tie band, logits within 1e-4 (the
reference's C++-vs-PyTorch drafter tolerance, ``tests/test_live_drafter.py:105-121``), draft
tokens, top-k ids and tree node tokens equal; the API invariants of the reference drafter tests
(``tests/test_live_drafter.py:34-73``: draft = teacher-forced chain, no mutation, exact rollback)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from lngram_hip import workloads as wl
from oracle import drafting as od
from oracle.cdrafter import CppDrafterPort

TAU = 2e-5
KINDS = ["sdb", "sdc"]


def _bundle(kind: str, seed: int = 5):
    w = {"sdb": wl.TINY_DRAFT, "sdc": wl.TINY_DRAFT_SSM}[kind]
    cfg, t = wl.build_draft_bundle(w, seed=seed)
    g = torch.Generator().manual_seed(9)
    for k in ("router_prev_norm", "router_cur_norm", "q_norm", "out_norm", "mem_norm"):
        t[k] = (1 + 0.2 * torch.randn(t[k].shape, generator=g)).to(t[k].dtype)
    return cfg, t


def _toks(cfg, n, seed=1):
    return torch.randint(0, cfg["vocab"], (n,), generator=torch.Generator().manual_seed(seed)).tolist()


@pytest.mark.parametrize("kind", KINDS)
def test_trace_codes_and_logits(kind):
    cfg, t = _bundle(kind)
    toks = _toks(cfg, 40)
    o = od.DrafterOracle(cfg, t)
    want_c, want_l = o.trace(toks)
    c = CppDrafterPort(cfg, t, threads=3)
    got_c, got_l = c.trace(toks)
    assert (got_c != want_c).mean() < 1e-2                  # own codes: flips only at near-ties
    # logits given identical codes
    got_c2, got_l2 = c.trace(toks, codes=want_c)
    assert np.array_equal(got_c2, want_c)
    assert np.abs(got_l2 - want_l).max() < 1e-4


@pytest.mark.parametrize("online", [False, True])
@pytest.mark.parametrize("kind", KINDS)
def test_draft_and_tree_match_oracle(kind, online):
    cfg, t = _bundle(kind)
    toks = _toks(cfg, 60, seed=2)
    o = od.DrafterOracle(cfg, t, online=online)
    o.commit(toks)
    codes = o.committed_codes()
    c = CppDrafterPort(cfg, t, threads=2, online=online)
    c.commit(toks, codes=codes)
    a, b = o.draft(4, hyp=toks[:0], topk=3), c.draft(4, topk=3)
    assert a.tokens == b.tokens
    assert np.array_equal(a.topk_ids, b.topk_ids)
    assert np.abs(a.topk_logits - b.topk_logits).max() < 1e-4
    spec = od.TreeSpec((-1, 0, 1, 2, 3, 0, 5, 6, 7, 1, 9, 10, 2, 12, 3, 0),
                       (0, 0, 0, 0, 0, 1, 0, 0, 0, 1, 0, 0, 1, 0, 1, 2))
    assert od.draft_tree(o, spec) == c.draft_tree(spec)


def test_api_invariants():
    cfg, t = _bundle("sdb")
    toks = _toks(cfg, 30, seed=3)
    c = CppDrafterPort(cfg, t, threads=1)
    c.commit(toks[:20])
    before = c.length
    d = c.draft(5, hyp=toks[20:22], topk=2, last_codes=True)
    assert c.length == before                               # drafting never mutates committed state
    assert d.codes.shape == (2 + 5, cfg["routes"])
    # draft = teacher-forced chain: committing the drafted tokens reproduces the next draft
    c2 = CppDrafterPort(cfg, t, threads=4)
    c2.commit(toks[:20] + toks[20:22] + d.tokens[:2])
    assert c2.draft(1).tokens[0] == d.tokens[2]
    c.commit(toks[20:25])
    c.truncate(20)                                          # exact rollback
    assert c.length == 20 and c.draft(5, hyp=toks[20:22], topk=2).tokens == d.tokens
    with pytest.raises(ValueError):
        c.truncate(21)
    with pytest.raises(RuntimeError):
        c.commit([cfg["vocab"]])
