"""The oracle's draft-tree verification pieces on the CPU (test infrastructure checking test
infrastructure): ``oracle.memory.ssm_tree`` (``drafting/tree.py:153-161``) and
``oracle.memory.tree_memory_forward`` (the memory block of ``tree_verify_step``, ``:179-196``).

Pins, none of them the formula under test retyped:
- a chain tree reduces to the pinned sequence functions (``ssm_scan``, ``memory_forward``);
- hand-computed states of a four-node tree;
- the path-sequence formulation of ``tree_memory_forward`` against a second, literal restatement
  of the reference's construction: code windows from ``tree_ngram_codes``, route tokens with the
  invalid slots as their own segment, the conv over ``tree_slots`` windows of normalised rows.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from oracle import drafting as od
from oracle import memory as om

PARENT = (-1, 0, 1, 0, 3, 1, 5, 2)
TREE16 = (-1, 0, 1, 2, 3, 0, 5, 6, 7, 1, 9, 10, 2, 12, 3, 0)


def test_tree_paths():
    assert om.tree_paths(PARENT) == [[0], [0, 1], [0, 1, 2], [0, 3], [0, 3, 4], [0, 1, 5], [0, 1, 5, 6],
                                     [0, 1, 2, 7]]
    for i in range(len(TREE16)):
        assert om.tree_paths(TREE16)[i] == od.tree_path(TREE16, i)


def test_ssm_tree_hand_values():
    a = np.array([0.5])
    u = np.array([4.0, 8.0, 0.0, 2.0]).reshape(1, 4, 1)
    s = om.ssm_tree(a, u, (-1, 0, 0, 1), s_root=np.array([[2.0]]))
    # s0 = .5*2 + .5*4 = 3; s1 = .5*3 + .5*8 = 5.5; s2 = .5*3 + 0 = 1.5; s3 = .5*5.5 + .5*2 = 3.75
    assert s[0, :, 0].tolist() == [3.0, 5.5, 1.5, 3.75]
    assert om.ssm_tree(a, u, (-1, 0, 0, 1))[0, 0, 0] == 2.0      # zero root state


def test_ssm_tree_chain_and_paths_equal_scan():
    rng = np.random.default_rng(0)
    a = rng.uniform(0.5, 0.99, 6)
    u = rng.standard_normal((2, len(TREE16), 6))
    s0 = rng.standard_normal((2, 6))
    chain = tuple(range(-1, len(TREE16) - 1))
    np.testing.assert_allclose(om.ssm_tree(a, u, chain, s0), om.ssm_scan(a, u, s0), rtol=0, atol=1e-14)
    st = om.ssm_tree(a, u, TREE16, s0)
    for i, path in enumerate(om.tree_paths(TREE16)):
        np.testing.assert_allclose(st[:, i], om.ssm_scan(a, u[:, path], s0)[:, -1], rtol=0, atol=1e-14)


def _layer(seed=0, d=32, routes=6, mem_dim=16, heads=4, kv=2, hd=8):
    g = torch.Generator().manual_seed(seed)
    cfg = om.MemCfg(d, routes, mem_dim, heads, kv, hd, eps=1e-6)
    p = {f"tables.ngram_{o}.weight": torch.randn(routes * 16 ** o, mem_dim, generator=g, dtype=torch.float64)
         for o in cfg.orders}
    p["readout_q_proj.weight"] = torch.randn(heads * hd, d, generator=g, dtype=torch.float64) * 0.2
    p["readout_query_norm.weight"] = 1 + 0.1 * torch.randn(d, generator=g, dtype=torch.float64)
    p["readout_memory_norm.weight"] = 1 + 0.1 * torch.randn(2 * mem_dim, generator=g, dtype=torch.float64)
    p["readout_kv_proj.weight"] = torch.randn(2 * kv * hd, 2 * mem_dim, generator=g, dtype=torch.float64) * 0.2
    p["readout_o_proj.weight"] = torch.randn(d, heads * hd, generator=g, dtype=torch.float64) * 0.2
    p["short_conv.norm.weight"] = 1 + 0.1 * torch.randn(d, generator=g, dtype=torch.float64)
    p["short_conv.conv.weight"] = torch.randn(d, 1, cfg.conv_kernel, generator=g, dtype=torch.float64) * 0.3
    return cfg, p, g


def _literal_tree_block(p, cfg, h_hist, codes_hist, h_nodes, codes_nodes, parent):
    """tree.py:179-196 step by step: windows along ancestors for the lookup and for the conv,
    the history's conv inputs from its own sequence forward."""
    b, L, d = h_hist.shape
    n = len(parent)
    tables = {o: p[f"tables.ngram_{o}.weight"] for o in cfg.orders}
    w_o = p["readout_o_proj.weight"]
    # the cached conv inputs of the history (RMSNorm'd o-proj rows of the history's own forward)
    q_h = om.project_query(p, cfg, h_hist)
    head_h = om.manual_gqa(cfg, q_h, *om.project_memory(p, cfg, om.route_tokens(tables, codes_hist, cfg.orders,
                                                                                 cfg.bits)))
    mixed_h = F.linear(head_h.reshape(b, L, cfg.q_heads * cfg.head_dim), w_o)
    # the nodes: n-gram windows along the ancestors, then the history (hist = 2)
    ctx, ok = od.tree_ngram_codes(parent, codes_nodes, codes_hist[:, max(0, L - 2):L], 2)
    seg = np.broadcast_to(ok.astype(np.int32)[None], ctx.shape[:3]).reshape(b * n, 3)
    tok = om.route_tokens(tables, ctx.reshape(b * n, 3, -1), cfg.orders, cfg.bits, segment_ids=seg)[:, -1]
    tok = tok.reshape(b, n, cfg.routes, -1)
    head_n = om.manual_gqa(cfg, om.project_query(p, cfg, h_nodes), *om.project_memory(p, cfg, tok))
    mixed_n = F.linear(head_n.reshape(b, n, cfg.q_heads * cfg.head_dim), w_o)
    # conv over each node's ancestor window of normalised rows (zero where the window runs out)
    ci = om.rms_norm_v2(torch.cat((mixed_h, mixed_n), 1), p["short_conv.norm.weight"], cfg.eps)
    lp = (cfg.conv_kernel - 1) * cfg.conv_dilation
    idx, okc = od.tree_slots(parent, L, lp)
    win = ci[:, torch.as_tensor(idx)] * torch.as_tensor(okc)[None, :, :, None].to(ci.dtype)
    y = F.conv1d(win.reshape(b * n, lp + 1, d).transpose(1, 2), p["short_conv.conv.weight"], None, 1, 0,
                 cfg.conv_dilation, d)
    return mixed_n + F.silu(y.transpose(1, 2).reshape(b, n, d))


def test_tree_memory_forward_matches_literal_restatement_and_chain():
    cfg, p, g = _layer()
    for L, parent in ((12, TREE16), (12, PARENT), (1, PARENT), (0, PARENT)):
        n = len(parent)
        h_hist = torch.randn(2, L, cfg.d_model, generator=g, dtype=torch.float64)
        h_nodes = torch.randn(2, n, cfg.d_model, generator=g, dtype=torch.float64)
        codes_hist = torch.randint(0, 16, (2, L, cfg.routes), generator=g).numpy()
        codes_nodes = torch.randint(0, 16, (2, n, cfg.routes), generator=g).numpy()
        got = om.tree_memory_forward(p, cfg, h_hist, codes_hist, h_nodes, codes_nodes, parent)
        want = _literal_tree_block(p, cfg, h_hist, codes_hist, h_nodes, codes_nodes, parent)
        assert om.rel_err(got, want) < 1e-12, (L, parent)
    # a chain tree is the sequence itself
    chain = tuple(range(-1, 7))
    h_hist = torch.randn(1, 10, cfg.d_model, generator=g, dtype=torch.float64)
    h_nodes = torch.randn(1, 8, cfg.d_model, generator=g, dtype=torch.float64)
    c_hist = torch.randint(0, 16, (1, 10, cfg.routes), generator=g).numpy()
    c_nodes = torch.randint(0, 16, (1, 8, cfg.routes), generator=g).numpy()
    got = om.tree_memory_forward(p, cfg, h_hist, c_hist, h_nodes, c_nodes, chain)
    full = om.memory_forward(p, cfg, torch.cat((h_hist, h_nodes), 1), np.concatenate((c_hist, c_nodes), 1))
    assert om.rel_err(got, full[:, 10:]) < 1e-12
