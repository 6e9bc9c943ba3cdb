"""Cached decoding of the memory layer on the GPU (``ffnmem.infer``: ``memory_step``,
``static_memory_step``; ``DepthwiseCausalConv.forward_incremental``), the checks of the
reference's ``tests/test_infer.py:38-65`` restricted to the memory layer: a prefill and steps of
mixed sizes reproduce the whole-sequence forward, a truncated state recomputes the same tail,
and a HIP-graph capture of the fixed-shape step replays the eager step at any cached length.

fp32 (tiny layer, materialised readout) and the bf16 SB shape with the fused readout run the same
kernels in both forms: equal bit for bit.  The bf16 whole-sequence forward of fewer than 1024
tokens takes the conv's row statistics from the output projection's epilogue (a different
summation order than the conv's own), so there the outputs are compared at bf16 tolerance and
the codes exactly.
"""

from __future__ import annotations

import pytest
import torch

from ffnmem.infer import DecodeState, memory_codes, memory_model, memory_step, router_input_at, ssm_continue, \
    static_memory_step
from ffnmem.memory.ssm import DiagonalSSM
from lngram_hip import ops
from lngram_hip import workloads as wl
from oracle import memory as om

pytestmark = pytest.mark.gpu


def _layer(w, dev):
    mem = wl.build_memory(w, seed=0, device=dev)
    h = wl.make_hidden(w, seed=1, device=dev)
    h_norm = ops.rmsnorm(h, torch.ones(w.d_model, dtype=w.dtype, device=dev), w.norm_eps)
    return mem, h, h_norm


def _decode(mem, h, h_norm, cuts):
    model = memory_model(mem)
    b, t, _ = h.shape
    st = DecodeState.empty(model, b, t)
    outs = []
    for a, e in zip(cuts[:-1], cuts[1:]):
        codes = memory_codes(model, 0, st, h_norm=h_norm[:, a:e])
        outs.append(memory_step(model, 0, st, h[:, a:e], codes))
        st.length = e
    return torch.cat(outs, 1), st


def test_fp32_prefill_and_steps_equal_full_forward(dev):
    w = wl.TINY.with_shape(2, 32)
    mem, h, h_norm = _layer(w, dev)
    with torch.no_grad():
        full = mem(h, h_norm)
        _, codes = mem.route_codes(h_norm)
        for cuts in ([0, 32], [0, 5, 8, 11, 14, 17, 20, 23, 26, 29, 32], [0, 1, 2, 3, 16, 32]):
            got, st = _decode(mem, h, h_norm, cuts)
            assert torch.equal(got, full), cuts
            assert torch.equal(st.codes[0], codes.to(torch.uint8))


def test_bf16_sb_shape_steps_match_full_forward(dev):
    w = wl.SB.with_shape(2, 40)
    mem, h, h_norm = _layer(w, dev)
    with torch.no_grad():
        full = mem(h, h_norm)
        _, codes = mem.route_codes(h_norm)
        got, st = _decode(mem, h, h_norm, [0, 7, 8, 9, 24, 40])
    assert torch.equal(st.codes[0], codes.to(torch.uint8))
    assert om.rel_err(got.float().cpu(), full.float().cpu()) < 5e-3
    assert (got == full).float().mean().item() > 0.98
    # against the bf16 oracle of the same codes
    sd = {k: v.detach().cpu() for k, v in mem.state_dict().items()}
    p = {k[len("module."):]: v for k, v in sd.items() if k.startswith("module.")}
    cfg = om.MemCfg(w.d_model, w.routes, w.mem_dim, w.q_heads, w.kv_heads, w.head_dim, eps=w.norm_eps)
    ref = om.memory_forward(p, cfg, h.cpu(), codes.cpu().numpy().astype("int32"))
    assert om.rel_err(got.float().cpu(), ref) < 2e-2


def test_step_with_route_codes_context_matches_oracle(dev):
    # memory_step(route_codes_ctx=...) (infer.py:152-182): the lookup of the new positions reads the
    # given code context [B, n + H, R] (here a history that differs from the cache) instead of the
    # cached codes, and the conv reads the cached rows in position order, as the reference's does.
    # The oracle: heads of the first L positions from the cached codes, heads of the new positions
    # from the context's n-grams, then one finish (o-proj + conv) over the whole sequence.
    w = wl.TINY.with_shape(2, 24)
    mem, h, h_norm = _layer(w, dev)
    model = memory_model(mem)
    L, n, hist = 20, 4, 2
    gen = torch.Generator().manual_seed(8)
    with torch.no_grad():
        st = DecodeState.empty(model, 2, 24)
        codes_a = memory_codes(model, 0, st, h_norm=h_norm[:, :L])
        memory_step(model, 0, st, h[:, :L], codes_a)
        st.length = L
        codes_new = torch.randint(0, 16, (2, n, w.routes), generator=gen, dtype=torch.uint8).to(dev)
        ctx_hist = torch.randint(0, 16, (2, hist, w.routes), generator=gen, dtype=torch.uint8).to(dev)
        ctx = torch.cat((ctx_hist, codes_new), 1)
        got = memory_step(model, 0, st, h[:, L:], codes_new, route_codes_ctx=ctx)
    assert torch.equal(st.codes[0][:, L:L + n], codes_new)
    sd = {k: v.detach().cpu() for k, v in mem.state_dict().items()}
    prm = {k[len("module."):]: v for k, v in sd.items() if k.startswith("module.")}
    cfg = om.MemCfg(w.d_model, w.routes, w.mem_dim, w.q_heads, w.kv_heads, w.head_dim, eps=w.norm_eps)
    h64 = h.cpu().double()
    p64 = {k: v.double() for k, v in prm.items()}
    tables = {o: p64[f"tables.ngram_{o}.weight"] for o in cfg.orders}
    q = om.project_query(p64, cfg, h64)
    tok_a = om.route_tokens(tables, codes_a.cpu().numpy(), cfg.orders, cfg.bits)
    tok_b = om.route_tokens(tables, ctx.cpu().numpy(), cfg.orders, cfg.bits, target_length=n)
    head_a = om.manual_gqa(cfg, q[:, :L], *om.project_memory(p64, cfg, tok_a))
    head_b = om.manual_gqa(cfg, q[:, L:], *om.project_memory(p64, cfg, tok_b))
    want = om.finish(p64, cfg, torch.cat((head_a, head_b), 1))[:, L:]
    assert om.rel_err(got.cpu().double(), want) < 1e-5
    # and the context matters: the cached history gives another output
    with torch.no_grad():
        st.length = L
        other = memory_step(model, 0, st, h[:, L:], codes_new)
    assert not torch.equal(other, got)


@pytest.mark.parametrize("shape", ["tiny", "sb"])
def test_truncate_then_recompute(dev, shape):
    w = (wl.TINY if shape == "tiny" else wl.SB).with_shape(1, 24)
    mem, hx, hnx = _layer(w, dev)
    gen = torch.Generator().manual_seed(5)
    hy = hx.clone()
    hy[:, 14:] = torch.randn(1, 10, w.d_model, generator=gen).to(w.dtype).to(dev)
    hny = ops.rmsnorm(hy, torch.ones(w.d_model, dtype=w.dtype, device=dev), w.norm_eps)
    model = memory_model(mem)
    st = DecodeState.empty(model, 1, 24)
    with torch.no_grad():
        for a, e in ((0, 12), (12, 20)):           # the second block is "rejected"
            memory_step(model, 0, st, hx[:, a:e], memory_codes(model, 0, st, h_norm=hnx[:, a:e]))
            st.length = e
        st.truncate(14)                             # keep 2 of it (x and y agree before 14)
        tail = memory_step(model, 0, st, hy[:, 14:], memory_codes(model, 0, st, h_norm=hny[:, 14:]))
        ref, _ = _decode(mem, hy, hny, [0, 14, 24])
    assert torch.equal(tail, ref[:, 14:])
    assert st.epoch == 1


@pytest.mark.parametrize("shape", ["tiny", "sb"])
def test_graph_captured_static_step_replays_eager(dev, shape):
    w = (wl.TINY if shape == "tiny" else wl.SB).with_shape(1, 48)
    mem, h, h_norm = _layer(w, dev)
    n = 4
    model = memory_model(mem)
    with torch.no_grad():
        eager, _ = _decode(mem, h, h_norm, [0, 16, 20, 24, 28, 32])
        st = DecodeState.empty(model, 1, 48)
        memory_step(model, 0, st, h[:, :16], memory_codes(model, 0, st, h_norm=h_norm[:, :16]))
        st.length = 16
        h_buf = torch.empty(1, n, w.d_model, dtype=w.dtype, device=dev)
        hn_buf = torch.empty_like(h_buf)
        L_t = torch.full((), 16, dtype=torch.int32, device=dev)

        def step():
            # the codes go from the router straight into the code cache (bf16) or through index_copy_
            return static_memory_step(model, 0, st, h_buf, None, L_t, router_x=hn_buf)

        # eager warm-up on a side stream writes past the cached length only, then capture
        h_buf.copy_(h[:, 16:20])
        hn_buf.copy_(h_norm[:, 16:20])
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                step()
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = step()
        for L in (16, 20, 24, 28):
            h_buf.copy_(h[:, L:L + n])
            hn_buf.copy_(h_norm[:, L:L + n])
            L_t.fill_(L)
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager[:, L:L + n]), L
            st.length = L + n
            # eager work between replays
            static_memory_step(model, 0, st, h_buf, memory_codes(model, 0, st, h_norm=hn_buf), L_t)
            torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_conv_forward_incremental_chains_to_forward(dev, dtype):
    w = wl.SB.with_shape(2, 40) if dtype == torch.bfloat16 else wl.TINY.with_shape(2, 40)
    mem, h, _ = _layer(w, dev)
    conv = mem.module.short_conv
    x = h * 0.5
    with torch.no_grad():
        full = conv(x)
        hist, outs = None, []
        for a, e in ((0, 5), (5, 8), (8, 9), (9, 30), (30, 40)):
            o, hist = conv.forward_incremental(x[:, a:e], hist)
            outs.append(o)
        assert hist.shape == (2, w.d_model, conv.left_padding)
    assert torch.equal(torch.cat(outs, 1), full)


def test_token_routed_decode_matches_full_forward(dev):
    # SD-B-style memory (embed2 router over E[x_{t-1}], E[x_t]) and an SD-C-style one with the
    # SSM state in its router: steps read the previous token / state from the cache
    for base in (wl.SDB, wl.SDC):
        w = base.with_shape(1, 40)
        mem, h, _ = _layer(w, dev)
        gen = torch.Generator().manual_seed(3)
        emb_tab = torch.nn.Embedding(w.vocab, w.d_model).to(dev, w.dtype)
        with torch.no_grad():
            emb_tab.weight.copy_((torch.randn(w.vocab, w.d_model, generator=gen) * 0.02).to(w.dtype))
        toks = torch.randint(0, w.vocab, (1, 40), generator=gen).to(dev)
        ssm = None
        if w.ssm_dim:
            torch.manual_seed(4)
            ssm = DiagonalSSM(w.d_model, w.ssm_dim).to(dev)
        model = memory_model(mem, tok_emb=emb_tab, ssm=ssm)
        with torch.no_grad():
            emb = emb_tab(toks)
            s_full = ssm(emb) if ssm is not None else None
            x = mem.router_features(emb, s_full)
            full = mem(h, None, router_in=x)
            _, codes_full = mem.route_codes(x)
            st = DecodeState.empty(model, 1, 40)
            outs = []
            for a, e in ((0, 9), (9, 10), (10, 27), (27, 40)):
                e_new = emb[:, a:e]
                s_new = ssm_continue(model, e_new, st.ssm[:, a - 1] if a > 0 else None) if ssm is not None else None
                rin = router_input_at(model, mem, st, e_new, s_new)
                codes = memory_codes(model, 0, st, router_in=rin)
                outs.append(memory_step(model, 0, st, h[:, a:e], codes))
                if s_new is not None:
                    st.ssm[:, a:e] = s_new
                st.tokens[:, a:e] = toks[:, a:e]
                st.length = e
            got = torch.cat(outs, 1)
        same = (st.codes[0] == codes_full.to(torch.uint8)).float().mean().item()
        if ssm is None:
            assert same == 1.0
            assert om.rel_err(got.float().cpu(), full.float().cpu()) < 5e-3
        else:
            # the carried SSM state rounds differently from the whole-sequence scan: router
            # logits near zero may flip a code
            assert same > 0.999
            assert om.rel_err(got.float().cpu(), full.float().cpu()) < 2e-2
