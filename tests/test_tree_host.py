"""Draft-tree structure helpers of the product (``drafting/tree.py``) on the CPU: the reference's own
known answers (``tests/test_live_tree.py:20-52``) and random trees against the oracle's
restatement of ``drafting/tree.py:65-127``, ``:243-257``."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from drafting import tree as dt
from oracle import drafting as od

PARENT = (-1, 0, 1, 0, 3, 1)  # 0 -> {1, 3}; 1 -> {2, 5}; 3 -> {4}


def test_reference_known_answers():
    m = dt.tree_attention_mask(PARENT, 2)
    expect = torch.tensor([[1, 1, 1, 0, 0, 0, 0, 0],
                           [1, 1, 1, 1, 0, 0, 0, 0],
                           [1, 1, 1, 1, 1, 0, 0, 0],
                           [1, 1, 1, 0, 0, 1, 0, 0],
                           [1, 1, 1, 0, 0, 1, 1, 0],
                           [1, 1, 1, 1, 0, 0, 0, 1]], dtype=torch.bool)
    assert torch.equal(m, expect)
    assert dt.tree_positions(PARENT, 5).tolist() == [5, 6, 7, 6, 7, 7]
    codes = torch.tensor([0, 10, 20, 30, 40, 50]).view(1, 6, 1)
    hist = torch.tensor([100, 101]).view(1, 2, 1)
    ctx, ok = dt.tree_ngram_codes(PARENT, codes, hist, 2)
    assert ctx[0, :, :, 0].tolist() == [[100, 101, 0], [101, 0, 10], [0, 10, 20], [101, 0, 30], [0, 30, 40],
                                        [0, 10, 50]]
    assert ok.all()
    ctx, ok = dt.tree_ngram_codes(PARENT, codes, None, 2)
    assert ok.tolist() == [[False, False, True], [False, True, True], [True, True, True], [False, True, True],
                           [True, True, True], [True, True, True]]
    assert ctx[0, 1, :, 0].tolist() == [0, 0, 10] and ctx[0, 4, :, 0].tolist() == [0, 30, 40]
    with pytest.raises(ValueError):
        dt.TreeSpec((-1, 2, 0), (0, 0, 0))
    with pytest.raises(ValueError):
        dt.TreeSpec((0, 0), (0, 0))
    with pytest.raises(ValueError):
        dt.TreeSpec((-1, 0), (0,))


def _random_parent(rng, n):
    return (-1,) + tuple(int(rng.integers(0, i)) for i in range(1, n))


@pytest.mark.parametrize("seed", range(6))
def test_structure_matches_oracle_on_random_trees(seed):
    rng = np.random.default_rng(seed)
    for n in (1, 2, 5, 16, 31):
        par = _random_parent(rng, n)
        assert dt.tree_depths(par) == od.tree_depths(par)
        for i in range(n):
            assert dt.tree_path(par, i) == od.tree_path(par, i)
        for L in (0, 1, 3, 7):
            assert (dt.tree_attention_mask(par, L).numpy() == od.tree_attention_mask(par, L)).all()
            for back in (0, 1, 2, 4):
                idx, ok = dt.tree_slots(par, L, back)
                widx, wok = od.tree_slots(par, L, back)
                assert (ok.numpy() == wok).all() and (idx.numpy() == widx).all()
        codes = torch.from_numpy(rng.integers(0, 16, (2, n, 3)))
        hist = torch.from_numpy(rng.integers(0, 16, (2, 4, 3)))
        for h in (None, hist):
            ctx, ok = dt.tree_ngram_codes(par, codes, h, 2)
            wctx, wok = od.tree_ngram_codes(par, codes.numpy(), None if h is None else h.numpy(), 2)
            assert (ctx.numpy() == wctx).all() and (ok.numpy() == wok).all()


class _ListDrafter:
    """A drafter whose candidates after a path are a fixed function of the path (no batched tree)."""

    def __init__(self):
        self.tokens = [11]

    def draft(self, gamma, hyp=(), topk=None, last_codes=False):
        base = (sum(hyp) * 7 + len(hyp) * 3) % 50
        ids = np.array([[base, base + 1, -1 if len(hyp) == 2 else base + 2]], np.int64)
        return od.DraftOut([int(ids[0, 0])], ids, np.zeros((1, 3), np.float32), np.zeros((0, 1), np.uint8))


@pytest.mark.parametrize("spec", [dt.tree16(), dt.default_tree(), dt.chain_tree(5)])
def test_draft_tree_matches_oracle(spec):
    got = dt.draft_tree(_ListDrafter(), spec)
    want = od.draft_tree(_ListDrafter(), od.TreeSpec(spec.parent, spec.rank))
    assert got == want
    assert got[0] == 11 and len(got) == spec.n
