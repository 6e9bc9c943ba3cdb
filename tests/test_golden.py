"""The oracle against the reference's own outputs (CPU).

The fixtures under ``tests/golden/`` were written by ``tests/golden/make_golden.py``, which ran
the reference modules on the inputs of ``tests/golden/recipe.py``.  Here the same inputs go
through the oracle:

- ``router_features`` (``router.py:50-68``): bit-exact in fp32 and bf16, both feature kinds,
  and the single-position ``step`` form at t = 0 (start vector) and t = 3;
- ``ssm_inputs`` and the scan (``ssm.py:37-91``) within fp32 rounding of the reference;
- the memory layer forward (``wrapper.py:103-125``): the tiny fp32 layer within 1e-5 and the
  bf16 layer at the SB widths against the reference's bf16 rounding sequence;
- the drafter (``cpu_drafter.py:147-289``): codes bit-exact, logits within 1e-5 norm-relative
  (fp64 oracle) of the reference's fp32, top-k ids equal, and the sketch shortlist identical;
- the online-count mix (``drafters.py:117-142``) within 2e-7 of the reference's fp32, plus a
  hand-computed mix weight.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import drafting as od
from oracle import memory as om

GOLD = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLD))
import recipe  # noqa: E402


def load(name: str) -> dict:
    with np.load(GOLD / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


# ------------------------------------------------------------------ router features
@pytest.mark.parametrize("kind", ["embed2", "embed2_ssm"])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_router_features_match_reference(kind, dt):
    g = load("router_features")
    d, n, b, t = 64, 16, 2, 6
    p = recipe.state({"prev_norm.weight": (d,), "cur_norm.weight": (d,), "start": (d,)}, 11)
    dtype = torch.bfloat16 if dt == "bf16" else torch.float32
    emb = torch.from_numpy(recipe.normal("rf_emb", (b, t, d))).to(dtype)
    s = torch.from_numpy(recipe.normal("rf_ssm", (b, t, n))) if kind == "embed2_ssm" else None
    w = {k: torch.from_numpy(v).to(dtype) for k, v in p.items()}
    got = om.router_features(emb, w["start"], w["prev_norm.weight"], w["cur_norm.weight"], 1e-5, s)
    key = f"{kind}_{dt}"
    want = bf16(g[f"{key}_out"]) if dt == "bf16" else torch.from_numpy(g[f"{key}_out"])
    assert torch.equal(got, want)
    # step (router.py:61-68) at t = 0 (start stands in for E[x_{-1}]) and t = 3 equals the sequence form
    for t_i, k in ((0, "step0"), (3, "step3")):
        st = bf16(g[f"{key}_{k}"]) if dt == "bf16" else torch.from_numpy(g[f"{key}_{k}"])
        assert torch.equal(got[:, t_i], st)


def test_router_features_closed_form():
    """Independent of both restatements: a constant row c·1 normalises to sign(c)·1 (times the
    weight), and the first position reads the start vector, not a token."""
    d = 32
    emb = torch.full((1, 3, d), -2.5, dtype=torch.float64)
    emb[0, 1] = 4.0
    start = torch.full((d,), 0.5, dtype=torch.float64)
    pw = torch.linspace(0.5, 1.5, d, dtype=torch.float64)
    cw = torch.linspace(2.0, 1.0, d, dtype=torch.float64)
    out = om.router_features(emb, start, pw, cw, 0.0)
    np.testing.assert_allclose(out[0, 0, :d], pw, rtol=1e-12)           # start = 0.5·1 -> +1
    np.testing.assert_allclose(out[0, 1, :d], -pw, rtol=1e-12)          # previous token -2.5·1 -> -1
    np.testing.assert_allclose(out[0, 1, d:], cw, rtol=1e-12)           # current 4·1 -> +1
    np.testing.assert_allclose(out[0, 2, :d], pw, rtol=1e-12)
    np.testing.assert_allclose(out[0, 2, d:], -cw, rtol=1e-12)


# ------------------------------------------------------------------ SSM
def test_ssm_inputs_and_scan_match_reference():
    g = load("ssm")
    d, n, b, t = 48, 16, 2, 21
    p = recipe.state({"norm.weight": (d,), "w_in.weight": (n, d), "theta": (n,)}, 12)
    emb = torch.from_numpy(recipe.normal("ssm_emb", (b, t, d)))
    u = om.ssm_inputs(emb, torch.from_numpy(p["norm.weight"]), torch.from_numpy(p["w_in.weight"]), 1e-5)
    assert om.rel_err(u, g["u"]) < 1e-6
    a = torch.sigmoid(torch.from_numpy(g["theta"]).float())
    s = om.ssm_scan(a.numpy(), g["u"])
    for k in ("s", "sequential", "chunked4"):
        assert om.rel_err(g[k], s) < 1e-5, k
    np.testing.assert_allclose(g["steps"], s[:, :3], rtol=0, atol=1e-6)


# ------------------------------------------------------------------ memory layer
def _memory_params(spec: dict, base: int) -> tuple[dict, om.MemCfg]:
    d, c = spec["d_model"], spec["cfg"]
    cfg = om.MemCfg(d, c["routes"], c["mem_dim"], c["q_heads"], c["kv_heads"], c["head_dim"])
    inner, kh = c["q_heads"] * c["head_dim"], c["kv_heads"] * c["head_dim"]
    shapes = {f"module.tables.ngram_{n}.weight": (cfg.routes * 16 ** n, cfg.mem_dim) for n in cfg.orders}
    shapes.update({
        "module.readout_query_norm.weight": (d,), "module.readout_memory_norm.weight": (cfg.route_token_dim,),
        "module.readout_q_proj.weight": (inner, d), "module.readout_kv_proj.weight": (2 * kh, cfg.route_token_dim),
        "module.readout_o_proj.weight": (d, inner), "module.short_conv.norm.weight": (d,),
        "module.short_conv.conv.weight": (d, 1, 4), "router.weight": (cfg.routes * 4, d)})
    raw = recipe.state(shapes, base)
    p = {(k[len("module."):] if k.startswith("module.") else k): torch.from_numpy(v) for k, v in raw.items()}
    return p, cfg


def test_memory_tiny_fp32_matches_reference():
    g = load("memory_tiny_fp32")
    p, cfg = _memory_params(recipe.TINY_MEM, 21)
    h = torch.from_numpy(recipe.normal("memory_tiny_fp32_h", (2, 16, cfg.d_model)))
    h_norm = torch.from_numpy(g["h_norm"])
    q = om.router_logits(h_norm, p["router.weight"], torch.float32)
    assert om.rel_err(q, g["q_logits"]) < 1e-6
    clear = np.abs(g["q_logits"]) > 1e-5
    want_codes = om.pack_route_codes(q.numpy(), 4)
    tie = ~clear.reshape(*want_codes.shape, 4).all(-1)
    assert tie.sum() == 0 and (want_codes == g["codes"]).all()
    out32 = om.memory_forward(p, cfg, h, g["codes"], dtype=torch.float32)
    out64 = om.memory_forward(p, cfg, h.double(), g["codes"])
    assert om.rel_err(out32, g["out"]) < 1e-6
    assert om.rel_err(out64, g["out"]) < 1e-5


def test_memory_sb_bf16_rounding_matches_reference():
    g = load("memory_sb_bf16")
    p, cfg = _memory_params(recipe.SB_MEM, 22)
    h = torch.from_numpy(recipe.normal("memory_sb_bf16_h", (1, 24, cfg.d_model))).to(torch.bfloat16)
    h_norm = bf16(g["h_norm"])
    assert torch.equal(om.rms_norm(h, torch.ones(cfg.d_model, dtype=torch.bfloat16), 1e-5), h_norm)
    q = om.router_logits(h_norm, p["router.weight"].to(torch.bfloat16), torch.float32)
    assert om.rel_err(q, g["q_logits"]) < 1e-6
    got = om.memory_forward(p, cfg, h, g["codes"], dtype=torch.bfloat16)
    want = bf16(g["out"])
    # the reference's bf16 rounding sequence, step for step: equal to the last bit
    assert torch.equal(got, want), om.rel_err(got, want)
    # and the fp64 restatement is within the bf16 tolerance of it
    assert om.rel_err(om.memory_forward(p, cfg, h.double(), g["codes"]), want) < 2e-2


# ------------------------------------------------------------------ drafter
DRAFTERS = ["drafter_sdb", "drafter_sdc", "drafter_sdb_sketch", "drafter_sdc_sketch"]


def _drafter(name: str, dtype=torch.float64) -> od.DrafterOracle:
    kind = name.split("_")[1]
    cfg = recipe.drafter_config(kind, sketch_k=4 if name.endswith("sketch") else 0, cap=6)
    arrays = recipe.drafter_arrays(cfg, 31)
    tensors = {k: torch.from_numpy(np.asarray(v).astype(np.int32) if v.dtype in (np.uint16, np.uint32) else v)
               for k, v in arrays.items()}
    return od.DrafterOracle(cfg, tensors, topk=3, dtype=dtype)


def _logit_err(got: np.ndarray, want: np.ndarray) -> float:
    ok = np.isfinite(want)
    assert (np.isfinite(got) == ok).all()
    return float(np.linalg.norm(got[ok] - want[ok]) / np.linalg.norm(want[ok]))


@pytest.mark.parametrize("name", DRAFTERS)
def test_drafter_trace_matches_reference(name):
    g = load(name)
    o = _drafter(name)
    c, ids, lg = o.trace_readout(g["tokens"], full=True)
    assert (c == g["full_codes"]).all()
    assert _logit_err(lg, g["full_logits"]) < 1e-5
    if "sl_ids" in g:
        c2, ids2, lg2 = o.trace_readout(g["tokens"])
        assert (ids2 == g["sl_ids"]).all()
        assert _logit_err(lg2, g["sl_logits"]) < 1e-5
    o32 = _drafter(name, torch.float32)
    _, _, lg32 = o32.trace_readout(g["tokens"], full=True)
    assert _logit_err(lg32, g["full_logits"]) < 1e-6


@pytest.mark.parametrize("name", DRAFTERS)
def test_drafter_draft_matches_reference(name):
    g = load(name)
    o = _drafter(name)
    o.commit(g["tokens"][:20])
    out = o.draft(4)
    assert out.tokens == g["draft_tokens"].tolist()
    assert (out.topk_ids == g["draft_ids"]).all() and (out.codes == g["draft_codes"]).all()
    assert _logit_err(out.topk_logits.astype(np.float64), g["draft_logits"]) < 1e-5
    out = o.draft(3, hyp=[int(g["tokens"][25]), int(g["tokens"][26])], last_codes=True)
    assert out.tokens == g["hyp_tokens"].tolist()
    assert (out.topk_ids == g["hyp_ids"]).all() and (out.codes == g["hyp_codes"]).all()
    assert _logit_err(out.topk_logits.astype(np.float64), g["hyp_logits"]) < 1e-5


# ------------------------------------------------------------------ online counts
@pytest.mark.parametrize("case", recipe.ONLINE_CASES, ids=[c[0] for c in recipe.ONLINE_CASES])
def test_online_counts_mix_matches_reference(case):
    # OnlineCounts(codes, x, orders, 4, V, kappa).mix (drafters.py:117-142), computed by the
    # reference in fp32; the oracle runs in fp64
    name, T, R, V, orders, kappa = case
    x = recipe.online_inputs(case)
    want = load("online_counts")[f"{name}_mix"].astype(np.float64)
    got = od.online_counts_mix(x["p"], x["codes"], x["x"], orders, 4, x["win"], x["real"], x["deadline"], kappa)
    got = got.numpy()
    assert np.abs(got - want).max() < 2e-7
    # the cases do what their windows say: unchanged rows (no match, no valid order, nothing
    # verified), and rows whose mix moved mass
    p = x["p"].astype(np.float64)
    for j in (3, 5, 6):
        assert np.abs(want[j] - p[j]).max() < 1e-7
    for j in (0, 1, 2):
        assert np.abs(want[j] - p[j]).max() > 1e-3


def test_online_mix_weight_hand_computed():
    # one route, orders 2 and 3, one matching pair: the 2-gram of the window (codes 1, 2) is the
    # row of pair t = 1, whose next token is x[2] = 12; the 3-gram (0, 1, 2) matches nothing.
    # n_eff = 1 / (1 route * 2 orders) = 1/2, lambda = n_eff / (n_eff + 1) = 1/3:
    # p' = 2/3 * p + 1/3 * onehot(12)
    codes = np.array([[1], [2], [3], [4]])
    x = np.array([10, 11, 12, 13])
    p = torch.full((1, 16), 1.0 / 16, dtype=torch.float64)
    win = np.array([[[0], [1], [2]]])
    real = np.ones((1, 3), bool)
    got = od.online_counts_mix(p, codes, x, (2, 3), 4, win, real, [2], kappa=1.0)
    want = torch.full((1, 16), (2.0 / 3.0) / 16, dtype=torch.float64)
    want[0, 12] += 1.0 / 3.0
    torch.testing.assert_close(got, want, rtol=0, atol=1e-15)
    # kappa 0.5: lambda = 0.5 / (0.5 + 0.5) = 1/2
    got = od.online_counts_mix(p, codes, x, (2, 3), 4, win, real, [2], kappa=0.5)
    want = torch.full((1, 16), 0.5 / 16, dtype=torch.float64)
    want[0, 12] += 0.5
    torch.testing.assert_close(got, want, rtol=0, atol=1e-15)


@pytest.mark.parametrize("name", ["drafter_sdb", "drafter_sdc"])
def test_drafter_online_mix_equals_counts_mix(name):
    # the drafter's per-cursor mix (keys = the first n_pairs committed pairs) is OnlineCounts.mix
    # at the cursor's window with deadline n_pairs - 1, which the fixture above pins
    g = load(name)
    o = _drafter(name)
    toks = np.concatenate([g["tokens"], g["tokens"][:12]])
    o.commit(toks)
    cur = o._cursor()
    codes = o.committed_codes()
    v = o.V
    p = torch.softmax(torch.from_numpy(recipe.normal(f"{name}_online_p", (v,))).double(), -1)
    win = codes[-3:][None]
    real = np.ones((1, 3), bool)
    for n_pairs in (5, 30, len(toks) - 1):
        got = o.online_mix(p, cur, n_pairs)
        want = od.online_counts_mix(p[None], codes, toks, o.ngrams, o.bits, win, real, [n_pairs - 1], o.kappa)[0]
        torch.testing.assert_close(got, want, rtol=0, atol=1e-14)
