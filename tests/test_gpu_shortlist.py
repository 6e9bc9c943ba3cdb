"""Sketch-shortlist drafting on the GPU (``lng_drafter_shortlist`` / ``lng_drafter_tree_shortlist``
through ``GpuDrafter``) against the reference's own outputs (``tests/golden/drafter_*_sketch.npz``,
written by ``RefDrafter`` from ``drafting/cpu_drafter.py``) and against the drafting oracle at
larger sketches (K = 16 slots, cap 64, duplicate tokens across routes and orders, positions
before the highest order, an empty sketch, a fallback list with repeats).

Shortlist ids, draft tokens, top-k ids and tree node tokens: equal.  Logits (fp32) against the
fp64 oracle or the reference's fp32: norm-relative error < 1e-5.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from drafting import tree as dtree
from drafting.gpu_drafter import GpuDrafter
from lngram_hip import workloads as wl
from oracle import drafting as od

GOLD = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLD))
import recipe  # noqa: E402

pytestmark = pytest.mark.gpu

GOLDEN = ["drafter_sdb_sketch", "drafter_sdc_sketch"]


def _golden(name: str) -> dict:
    z = np.load(GOLD / f"{name}.npz")
    return {k: z[k] for k in z.files}


def _rel(got, want) -> float:
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    ok = np.isfinite(want)
    assert (np.isfinite(got) == ok).all()
    return float(np.linalg.norm(got[ok] - want[ok]) / np.linalg.norm(want[ok]))


def _recipe_bundle(name: str):
    kind = name.split("_")[1]
    cfg = recipe.drafter_config(kind, sketch_k=4, cap=6)
    arrays = recipe.drafter_arrays(cfg, 31)
    tensors = {k: torch.from_numpy(np.asarray(v).astype(np.int32) if v.dtype in (np.uint16, np.uint32) else v)
               for k, v in arrays.items()}
    return cfg, tensors


@pytest.mark.parametrize("name", GOLDEN)
def test_shortlist_trace_and_drafts_match_reference(dev, name):
    g = _golden(name)
    cfg, t = _recipe_bundle(name)
    d = GpuDrafter((cfg, t), device=dev, max_len=64)
    assert d.cap == 6 and d.sketch is not None
    codes, ids, lg = d.trace(g["tokens"])
    np.testing.assert_array_equal(codes, g["full_codes"])
    np.testing.assert_array_equal(ids, g["sl_ids"])
    assert _rel(lg, g["sl_logits"]) < 1e-5
    _, ids_full, lg_full = d.trace(g["tokens"], full=True)
    assert ids_full.shape == g["full_logits"].shape
    assert _rel(lg_full, g["full_logits"]) < 1e-5
    d.commit(g["tokens"][:20])
    out = d.draft(4)
    assert out.tokens == g["draft_tokens"].tolist()
    np.testing.assert_array_equal(out.topk_ids, g["draft_ids"])
    np.testing.assert_array_equal(out.codes, g["draft_codes"])
    assert _rel(out.topk_logits, g["draft_logits"]) < 1e-5
    out = d.draft(3, hyp=[int(g["tokens"][25]), int(g["tokens"][26])], last_codes=True)
    assert out.tokens == g["hyp_tokens"].tolist()
    np.testing.assert_array_equal(out.topk_ids, g["hyp_ids"])
    np.testing.assert_array_equal(out.codes, g["hyp_codes"])
    assert _rel(out.topk_logits, g["hyp_logits"]) < 1e-5


def _sketch_bundle(kind: str, k: int = 16, cap: int = 64, seed: int = 11, fallback: int = 80):
    """TINY drafter bundle plus count sketches: ids from a small pool (so tokens repeat across
    slots, routes and orders), counts 0..5 (0 = empty), a fallback list with repeats."""
    w = {"sdb": wl.TINY_DRAFT, "sdc": wl.TINY_DRAFT_SSM}[kind]
    cfg, t = wl.build_draft_bundle(w, seed=5)
    gen = np.random.default_rng(seed)
    V, R, bits = cfg["vocab"], cfg["routes"], cfg["bits"]
    pool = gen.choice(V, size=48, replace=False)
    for n in cfg["ngrams"]:
        rows = R * (1 << (bits * n))
        t[f"sketch_ids_{n}"] = torch.from_numpy(pool[gen.integers(0, len(pool), (rows, k))].astype(np.int32))
        t[f"sketch_counts_{n}"] = torch.from_numpy(gen.integers(0, 6, (rows, k)).astype(np.int64))
    fb = np.concatenate([pool[:10], pool[:10], gen.choice(V, size=fallback - 20)])
    t["fallback"] = torch.from_numpy(fb.astype(np.int32))
    cfg = dict(cfg, sketch_k=k, shortlist_cap=cap)
    return cfg, t


@pytest.mark.parametrize("kind", ["sdb", "sdc"])
def test_shortlist_matches_oracle_with_repeats_and_fallback(dev, kind):
    cfg, t = _sketch_bundle(kind)
    toks = torch.randint(0, cfg["vocab"], (40,), generator=torch.Generator().manual_seed(6)).tolist()
    o = od.DrafterOracle(cfg, t, topk=3)
    assert o.cap == 64 and o.sk_ids
    oc, oi, ol = o.trace_readout(toks)
    d = GpuDrafter((cfg, t), device=dev, max_len=96)
    c, ids, lg = d.trace(toks, codes=oc)
    np.testing.assert_array_equal(ids, oi)
    assert _rel(lg, ol) < 1e-5
    # drafts over the shortlist after a committed context, with and without hypothetical tokens
    o.reset()
    o.commit(toks, codes=oc)
    d.commit(toks, codes=oc)
    for hyp, gamma, k, last in (((), 4, 3, False), (tuple(toks[5:7]), 3, 4, True), ((), 1, 1, False)):
        want = o.draft(gamma, hyp=hyp, topk=k, last_codes=last)
        got = d.draft(gamma, hyp=hyp, topk=k, last_codes=last)
        assert got.tokens == want.tokens, (hyp, gamma)
        np.testing.assert_array_equal(got.topk_ids, want.topk_ids)
        assert _rel(got.topk_logits, want.topk_logits) < 1e-5
        np.testing.assert_array_equal(got.codes, want.codes)
    # draft trees: every parent's children come from its shortlist
    for spec in (dtree.tree16(), dtree.default_tree()):
        want = od.draft_tree(o, od.TreeSpec(spec.parent, spec.rank))
        assert d.draft_tree(spec) == want
        node_tok, rt = d.tree_step(spec, route_tokens=True)
        assert node_tok.cpu().tolist() == want and rt.shape == (spec.n, cfg["routes"], d.dt)


@pytest.mark.parametrize("scale", [0, 40, 57])
def test_shortlist_totals_of_any_width(dev, scale):
    """Totals of a few bits (ties broken by id), near 2^45 (the radix select walks every byte of
    the key) and above 2^(64 - id bits) (the one-maximum-at-a-time path): the lists, drafts and
    logits equal the oracle's, through the trace (full-vocabulary logits) and through draft (the
    candidates scored from the hidden state)."""
    cfg, t = _sketch_bundle("sdb", k=8, cap=24, seed=17)
    gen = np.random.default_rng(23)
    for n in cfg["ngrams"]:
        c = t[f"sketch_counts_{n}"].numpy()
        wide = c * (np.int64(1) << scale) + (c > 0) * gen.integers(0, 4, c.shape)
        t[f"sketch_counts_{n}"] = torch.from_numpy(wide.astype(np.int64))
    toks = torch.randint(0, cfg["vocab"], (24,), generator=torch.Generator().manual_seed(8)).tolist()
    o = od.DrafterOracle(cfg, t, topk=3)
    oc, oi, ol = o.trace_readout(toks)
    d = GpuDrafter((cfg, t), device=dev, max_len=64)
    _, ids, lg = d.trace(toks, codes=oc)
    np.testing.assert_array_equal(ids, oi)
    assert _rel(lg, ol) < 1e-5
    o.reset()
    o.commit(toks, codes=oc)
    d.commit(toks, codes=oc)
    for hyp, gamma in (((), 4), (tuple(toks[3:5]), 2)):
        want = o.draft(gamma, hyp=hyp, topk=3)
        got = d.draft(gamma, hyp=hyp, topk=3)
        assert got.tokens == want.tokens
        np.testing.assert_array_equal(got.topk_ids, want.topk_ids)
        assert _rel(got.topk_logits, want.topk_logits) < 1e-5


def test_shortlist_edge_cases(dev):
    cfg, t = _sketch_bundle("sdb", cap=8, fallback=20)
    V = cfg["vocab"]
    toks = [3, 9, 27, 81]
    # an empty sketch and no fallback: every position scores the whole vocabulary (trace cut to cap)
    t0 = dict(t)
    for n in cfg["ngrams"]:
        t0[f"sketch_counts_{n}"] = torch.zeros_like(t[f"sketch_counts_{n}"])
    t0["fallback"] = torch.zeros(0, dtype=torch.int32)
    o = od.DrafterOracle(cfg, t0)
    oc, oi, ol = o.trace_readout(toks)
    d = GpuDrafter((cfg, t0), device=dev, max_len=16)
    _, ids, lg = d.trace(toks, codes=oc)
    np.testing.assert_array_equal(ids, oi)
    assert (ids == np.arange(8)[None]).all()
    assert _rel(lg, ol) < 1e-5
    o.commit(toks, codes=oc)
    d.commit(toks, codes=oc)
    want, got = o.draft(2, topk=3), d.draft(2, topk=3)
    assert got.tokens == want.tokens and (got.topk_ids == want.topk_ids).all()
    # only fallback tokens (empty sketch): the list is the fallback's first occurrences
    t1 = dict(t0)
    t1["fallback"] = torch.tensor([5, 5, 7, 1, 7, 2, 9, 11, 13, 2, 15], dtype=torch.int32)
    o1 = od.DrafterOracle(cfg, t1)
    oc1, oi1, ol1 = o1.trace_readout(toks)
    d1 = GpuDrafter((cfg, t1), device=dev, max_len=16)
    _, ids1, lg1 = d1.trace(toks, codes=oc1)
    np.testing.assert_array_equal(ids1, oi1)
    assert ids1[0].tolist() == [5, 7, 1, 2, 9, 11, 13, 15]
    assert _rel(lg1, ol1) < 1e-5
    # shortlist_cap=0 turns the shortlist off: full-vocabulary scores
    d2 = GpuDrafter((cfg, t), shortlist_cap=0, device=dev, max_len=16)
    assert d2.sketch is None
    _, ids2, _ = d2.trace(toks)
    assert ids2.shape == (len(toks), V)
    with pytest.raises(ValueError, match="online"):
        GpuDrafter((cfg, t), device=dev, online=True)


def test_sdc_bundle_shape_shortlist_runs_and_matches_oracle(dev):
    # the reference's published SD-C drafter configuration: R 181, V 32768, d 1024, bf16, sketch
    # K = 16 per row and order, shortlist cap 64 (2 x 181 x 16 = 5792 slots per position)
    w = wl.SDC_DRAFT
    cfg, t = wl.build_draft_bundle(w, seed=0)
    gen = np.random.default_rng(3)
    V, R, bits = cfg["vocab"], cfg["routes"], cfg["bits"]
    for n in cfg["ngrams"]:
        rows = R * (1 << (bits * n))
        t[f"sketch_ids_{n}"] = torch.from_numpy(gen.integers(0, 4096, (rows, 16)).astype(np.int32))
        t[f"sketch_counts_{n}"] = torch.from_numpy(gen.integers(0, 3, (rows, 16)).astype(np.int64))
    t["fallback"] = torch.from_numpy(gen.choice(V, size=64, replace=False).astype(np.int32))
    cfg = dict(cfg, sketch_k=16, shortlist_cap=64)
    ctx = wl.make_context(w, seed=0)[:256]
    g = GpuDrafter((cfg, t), device=dev, max_len=512)
    g.commit(ctx)
    codes = g.committed_codes()
    o = od.DrafterOracle(cfg, t)
    o.commit(ctx, codes=codes)
    want = o.draft(3, topk=3)
    got = g.draft(3, topk=3)
    assert got.tokens == want.tokens
    np.testing.assert_array_equal(got.topk_ids, want.topk_ids)
    assert _rel(got.topk_logits, want.topk_logits) < 1e-5
    # the trace of the last positions: the shortlists and their logits
    _, ids, lg = g.trace(ctx[-24:], codes=codes[-24:])
    o2 = od.DrafterOracle(cfg, t)
    _, oi, ol = o2.trace_readout(ctx[-24:], codes=codes[-24:])
    np.testing.assert_array_equal(ids, oi)
    assert _rel(lg, ol) < 1e-5
