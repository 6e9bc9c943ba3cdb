"""The memory block of draft-tree verification on the GPU (``tree_verify_step``,
``drafting/tree.py:141-202``): ``lng_causal_conv_slots`` (the conv over ancestor windows, :186-194),
``lng_ssm_tree`` (the parent-ordered SSM, :153-161), the token-router features of tree nodes
(:170-177) and ``ffnmem.infer.tree_memory_step`` (:179-196).

Each node's output must be what decoding its root path token by token gives: bit for bit against
``memory_step`` chains (the same kernels per token), and against the oracle's
``tree_memory_forward`` (fp64 for the fp32 layer, the bf16 restatement for the SB shape).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from drafting.tree import tree16, tree_slots
from ffnmem.infer import DecodeState, memory_codes, memory_model, memory_step, static_tree_memory_step, \
    tree_memory_step, tree_router_input, tree_ssm_states
from ffnmem.memory.ssm import DiagonalSSM
from lngram_hip import ops
from lngram_hip import workloads as wl
from oracle import memory as om

pytestmark = pytest.mark.gpu

PARENT = tree16().parent


def _slots(parent, L, back):
    s, ok = tree_slots(parent, L, back)
    return torch.where(ok, s, torch.full_like(s, -1)), ok


@pytest.mark.parametrize("L", [3, 20])
@pytest.mark.parametrize("case", ["bf16_k4d3", "f32_k4d3", "bf16_k3d2"])
def test_conv_slots_equal_sequence_conv_of_gathered_windows(dev, case, L):
    dt, d, k, dil = {"bf16_k4d3": (torch.bfloat16, 1024, 4, 3), "f32_k4d3": (torch.float32, 128, 4, 3),
                     "bf16_k3d2": (torch.bfloat16, 96, 3, 2)}[case]
    n, b = len(PARENT), 2
    g = torch.Generator().manual_seed(5)
    rows = (torch.randn(b, L + n + 3, d, generator=g) * 0.7).to(dt).to(dev)
    nw = (1 + 0.1 * torch.randn(d, generator=g)).to(dt).to(dev)
    cw = (torch.randn(d, 1, k, generator=g) * 0.4).to(dt).to(dev)
    back = (k - 1) * dil
    slots, ok = _slots(PARENT, L, back)
    got = ops.causal_conv_slots(rows, nw, cw, dil, 1e-6, slots, length=L + n)
    # each node's window as a sequence of its own (zero rows where it runs past position 0):
    # the sequence conv's output at the window's last position
    okd = ok.to(dev)
    win = torch.where(okd[None, :, :, None], rows[:, slots.clamp_min(0).to(dev)], torch.zeros((), dtype=dt, device=dev))
    want = ops.causal_conv(win.reshape(b * n, back + 1, d), nw, cw, dil, 1e-6)[:, -1].reshape(b, n, d)
    assert torch.equal(got, want)
    if L < back:
        assert not bool(ok.all())      # the padding slots were exercised
    # without the residual, and a slot past `length` reads a zero row
    got_nr = ops.causal_conv_slots(rows, nw, cw, dil, 1e-6, slots, length=L + n, residual=False)
    want_nr = ops.causal_conv(win.reshape(b * n, back + 1, d), nw, cw, dil, 1e-6, residual=False)[:, -1]
    assert torch.equal(got_nr, want_nr.reshape(b, n, d))
    cut = ops.causal_conv_slots(rows, nw, cw, dil, 1e-6, slots, length=L)   # the nodes' own rows out of range
    assert torch.equal(cut, ops.causal_conv_slots(torch.cat((rows[:, :L], torch.zeros_like(rows[:, L:])), 1), nw, cw,
                                                  dil, 1e-6, slots, length=L + n))


def test_conv_slots_rejects_bad_arguments(dev):
    rows = torch.zeros(1, 8, 64, dtype=torch.bfloat16, device=dev)
    w = torch.ones(64, 1, 4, dtype=torch.bfloat16, device=dev)
    nw = torch.ones(64, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        ops.causal_conv_slots(rows, nw, w, 3, 1e-6, torch.zeros(2, 9, dtype=torch.int32))   # needs 10 slots
    with pytest.raises(RuntimeError):
        ops.causal_conv_slots(rows, nw, w, 3, 1e-6, torch.zeros(2, 10, dtype=torch.int32), length=9)  # > S


@pytest.mark.parametrize("root", [True, False])
def test_ssm_tree_equals_scan_along_paths_and_oracle(dev, root):
    g = torch.Generator().manual_seed(6)
    n, b, c = len(PARENT), 2, 256
    a = (0.9 + 0.099 * torch.rand(c, generator=g)).to(dev)
    u = torch.randn(b, n, c, generator=g).to(dev)
    s_root = torch.randn(b, c, generator=g).to(dev) if root else None
    got = ops.ssm_tree(a, u, PARENT, s_root)
    for i, path in enumerate(om.tree_paths(PARENT)):
        assert torch.equal(got[:, i], ops.ssm_scan(a, u[:, path], s_root)[:, -1]), i
    want = om.ssm_tree(a.cpu().numpy(), u.cpu().numpy(), PARENT, None if s_root is None else s_root.cpu().numpy())
    assert om.rel_err(got.cpu().double(), torch.from_numpy(want)) < 1e-6


def _layer(w, dev):
    mem = wl.build_memory(w, seed=0, device=dev)
    h = wl.make_hidden(w, seed=1, device=dev)
    h_norm = ops.rmsnorm(h, torch.ones(w.d_model, dtype=w.dtype, device=dev), w.norm_eps)
    return mem, h, h_norm


def _params(mem):
    sd = {k: v.detach().cpu() for k, v in mem.state_dict().items()}
    return {k[len("module."):]: v for k, v in sd.items() if k.startswith("module.")}


@pytest.mark.parametrize("shape", ["tiny", "sb"])
def test_tree_memory_step_equals_chain_decode_and_oracle(dev, shape):
    n = len(PARENT)
    b, L = (2, 20) if shape == "tiny" else (1, 12)
    w = (wl.TINY if shape == "tiny" else wl.SB).with_shape(b, L + n)
    mem, h, h_norm = _layer(w, dev)
    model = memory_model(mem)
    with torch.no_grad():
        st = DecodeState.empty(model, b, L + n)
        codes_h = memory_codes(model, 0, st, h_norm=h_norm[:, :L])
        memory_step(model, 0, st, h[:, :L], codes_h)
        st.length = L
        st0 = st.index_select(torch.arange(b, device=dev))
        hn = h[:, L:]
        codes_n = memory_codes(model, 0, st, h_norm=h_norm[:, L:])
        got = tree_memory_step(model, 0, st, hn, codes_n, PARENT)
        assert torch.equal(st.codes[0][:, L:L + n], codes_n.to(torch.uint8))
        for i, path in enumerate(om.tree_paths(PARENT)):
            sti = st0.index_select(torch.arange(b, device=dev))
            for p in path:
                out = memory_step(model, 0, sti, hn[:, p:p + 1], codes_n[:, p:p + 1])
                sti.length += 1
            assert torch.equal(got[:, i:i + 1], out), i
    prm = _params(mem)
    cfg = om.MemCfg(w.d_model, w.routes, w.mem_dim, w.q_heads, w.kv_heads, w.head_dim, eps=w.norm_eps)
    ch = codes_h.cpu().numpy().astype(np.int64)
    cn = codes_n.cpu().numpy().astype(np.int64)
    if shape == "tiny":
        want = om.tree_memory_forward(prm, cfg, h[:, :L].cpu().double(), ch, hn.cpu().double(), cn, PARENT,
                                      dtype=torch.float64)
        assert om.rel_err(got.cpu().double(), want) < 1e-5
    else:
        want = om.tree_memory_forward(prm, cfg, h[:, :L].cpu(), ch, hn.cpu(), cn, PARENT)
        assert om.rel_err(got.float().cpu(), want.float()) < 2e-2


@pytest.mark.parametrize("shape", ["tiny", "sb"])
def test_static_tree_step_graph_replays_eager(dev, shape):
    # the fixed-shape tree step captured once in a HIP graph and replayed at other device-held
    # lengths (1, 2 and 9 cached positions included: history windows that run past position 0);
    # the caches are restored between replays (eager work between them) and every replay is held
    # to the eager step at that length
    n = len(PARENT)
    b, hist_len = (2, 12) if shape == "tiny" else (1, 12)
    w = (wl.TINY if shape == "tiny" else wl.SB).with_shape(b, hist_len + n)
    mem, h, h_norm = _layer(w, dev)
    model = memory_model(mem)
    with torch.no_grad():
        base = DecodeState.empty(model, b, hist_len + n)
        memory_step(model, 0, base, h[:, :hist_len], memory_codes(model, 0, base, h_norm=h_norm[:, :hist_len]))
        hn = h[:, hist_len:].contiguous()
        codes_n = memory_codes(model, 0, base, h_norm=h_norm[:, hist_len:])
        st = base.index_select(torch.arange(b, device=dev))
        L_t = torch.full((), hist_len, dtype=torch.int32, device=dev)
        static_tree_memory_step(model, 0, st, hn, codes_n, PARENT, L_t)      # warm: index tables built
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = static_tree_memory_step(model, 0, st, hn, codes_n, PARENT, L_t)
        for L in (hist_len, 9, 1, 2, hist_len):
            st.codes[0].copy_(base.codes[0])
            st.conv_in[0].copy_(base.conv_in[0])
            L_t.fill_(L)
            g.replay()
            torch.cuda.synchronize()
            ref = base.index_select(torch.arange(b, device=dev))
            ref.length = L
            want = tree_memory_step(model, 0, ref, hn, codes_n, PARENT)
            assert torch.equal(out, want), L
            assert torch.equal(st.codes[0][:, L:L + n], ref.codes[0][:, L:L + n])
            assert torch.equal(st.conv_in[0][:, L:L + n], ref.conv_in[0][:, L:L + n])


def test_tree_memory_step_rejects_bad_calls(dev):
    w = wl.TINY.with_shape(1, 8)
    mem, h, h_norm = _layer(w, dev)
    model = memory_model(mem)
    st = DecodeState.empty(model, 1, 8)
    codes = memory_codes(model, 0, st, h_norm=h_norm[:, :4])
    with pytest.raises(ValueError):
        tree_memory_step(model, 0, st, h[:, :4], codes, (-1, 0, 1))          # three parents, four nodes
    st.length = 6
    with pytest.raises(ValueError):
        tree_memory_step(model, 0, st, h[:, :4], codes, (-1, 0, 1, 1))       # cache full


@pytest.mark.parametrize("L", [0, 10])
def test_tree_router_input_and_states_match_path_sequences(dev, L):
    # SD-C-style memory (embed2_ssm router): each node's previous token is its parent's, its SSM
    # state continues its parent's; the root continues the last cached token and state
    n = len(PARENT)
    w = wl.SDC.with_shape(1, L + n)
    mem = wl.build_memory(w, seed=0, device=dev)
    g = torch.Generator().manual_seed(9)
    emb_tab = torch.nn.Embedding(w.vocab, w.d_model).to(dev, w.dtype)
    torch.manual_seed(4)
    ssm = DiagonalSSM(w.d_model, w.ssm_dim).to(dev)
    model = memory_model(mem, tok_emb=emb_tab, ssm=ssm)
    feats = mem.router_features
    with torch.no_grad():
        emb_tab.weight.copy_((torch.randn(w.vocab, w.d_model, generator=g) * 0.02).to(w.dtype))
        toks = torch.randint(0, w.vocab, (1, L + n), generator=g).to(dev)
        st = DecodeState.empty(model, 1, L + n)
        if L:
            st.ssm[:, :L] = ssm(emb_tab(toks[:, :L]))
            st.tokens[:, :L] = toks[:, :L]
            st.length = L
        e_nodes = emb_tab(toks[:, L:])
        s_new = tree_ssm_states(model, st, e_nodes, PARENT)
        rin = tree_router_input(model, mem, st, e_nodes, s_new, PARENT)
        u = ssm.inputs(e_nodes)
        s0 = st.ssm[:, L - 1] if L else None
        for i, path in enumerate(om.tree_paths(PARENT)):
            assert torch.equal(s_new[:, i], ops.ssm_scan(ssm.decay(), u[:, path], s0)[:, -1]), i
            seq, sseq = e_nodes[:, path], s_new[:, path]
            if L:
                seq = torch.cat((emb_tab(toks[:, L - 1:L]), seq), 1)
                sseq = torch.cat((st.ssm[:, L - 1:L], sseq), 1)
            want = om.router_features(seq.cpu(), feats.start.detach().cpu(), feats.prev_norm.weight.detach().cpu(),
                                      feats.cur_norm.weight.detach().cpu(), feats.prev_norm.eps,
                                      ssm_state=sseq.cpu())[:, -1]
            assert torch.equal(rin[:, i].cpu(), want), i
        # the codes of the nodes, then the memory block, run on these features
        codes = memory_codes(model, 0, st, router_in=rin)
        out = tree_memory_step(model, 0, st, mem.module.readout_q_proj.weight.new_zeros(1, n, w.d_model) +
                               0.5, codes, PARENT)
        assert out.shape == (1, n, w.d_model) and bool(torch.isfinite(out.float()).all())


@pytest.mark.parametrize("L", [0, 1, 5])
@pytest.mark.parametrize("on_device", [False, True])
def test_tree_windows_equal_index_formulation(dev, L, on_device):
    """``lng_tree_windows`` against the same windows built from torch index ops: the codes of each
    node's window over (the last 2 cached codes, the node codes), zero and not real where a history
    slot precedes position 0; the node codes cached at L .. L+n-1; the conv slots rel + L.  Lengths
    shorter than the history included, with the length on the host or in device memory."""
    B, R, n, hist, back = 2, 5, len(PARENT), 2, 9
    gen = torch.Generator().manual_seed(60 + L)
    cache = torch.randint(0, 16, (B, 40, R), generator=gen, dtype=torch.uint8).to(dev)
    codes = torch.randint(0, 16, (B, n, R), generator=gen, dtype=torch.int32).to(dev)
    idx, _ = tree_slots(PARENT, hist, hist)
    full, _ = tree_slots(PARENT, back + 1, back)
    idx, rel = idx.to(dev), (full - (back + 1)).to(torch.int32).to(dev)
    # the index formulation
    c8 = codes.to(torch.uint8)
    base = (L - hist) + torch.arange(hist, device=dev)
    seq = torch.cat((cache.index_select(1, base.clamp_min(0)), c8), 1)
    real = (idx >= hist) | ((idx - hist + L) >= 0)
    want_win = seq.index_select(1, idx.reshape(-1)).view(B * n, hist + 1, R) * \
        real[None].expand(B, n, hist + 1).reshape(B * n, hist + 1, 1).to(torch.uint8)
    want_real = real[None].expand(B, n, hist + 1).reshape(B * n, hist + 1)
    want_cache = cache.clone()
    want_cache[:, L:L + n] = c8
    L_dev = torch.tensor([L], dtype=torch.int32, device=dev) if on_device else None
    win, seg, val, slots = ops.tree_windows(cache, codes, idx.to(torch.int32), hist, 0 if on_device else L, L_dev,
                                            rel)
    torch.cuda.synchronize()
    assert torch.equal(win, want_win)
    assert torch.equal(seg, want_real.to(torch.int32)) and torch.equal(val, want_real.to(torch.uint8))
    assert torch.equal(cache, want_cache)
    assert torch.equal(slots, rel + L)
