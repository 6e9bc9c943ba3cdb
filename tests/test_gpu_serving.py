"""Serving layout and host-RAM row providers on the GPU (``serving.layout``, ``serving.prefetch``;
reference ``serving/layout.py``, ``serving/prefetch.py``), with the checks of the reference's
``tests/test_index_layout.py:48-80``, ``tests/test_serving_prefetch.py`` and
``tests/test_serving_spec.py`` applied to the memory layers' cached decode (``memory_decode``):

- the serving layout gives the v2 lookup's route tokens, its candidate blocks hold the next rows,
  and the permutation is an involution;
- decoding with the rows of B1 (exact gather from host RAM) and B4 (prefetched candidate blocks)
  equals decoding with the tables on the device bit for bit (tiny fp32 layer, SB-shape bf16 layer
  with the fused readout, two layers), including positions 0 and 1, a rollback and a new state;
- staged verify blocks return exactly the direct lookup's rows, and verify-block decoding equals
  the on-device decode;
- the row and byte accounting, offload / restore.
"""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import memory as om

from ffnmem.infer import DecodeState, memory_decode
from lngram_hip import ops
from lngram_hip import workloads as wl
from serving import layout as sl
from serving.prefetch import (BlockStager, CandidatePrefetcher, HostGather, HostTables, LayerTable, ZeroCopyGather,
                              offload_tables, restore_tables)

pytestmark = pytest.mark.gpu

VARIANTS = {"tiny": [wl.TINY], "sb": [wl.SB], "tiny_2mem": [wl.TINY, wl.TINY]}


def make(variant: str, dev, batch: int = 2, seq: int = 32):
    """A model of one or two memory layers (block 1 between them has none), with non-zero tables,
    and per layer its hidden states and router inputs for ``seq`` positions."""
    blocks, inputs = [], {}
    for i, w in enumerate(VARIANTS[variant]):
        ws = w.with_shape(batch, seq)
        mem = wl.build_memory(ws, seed=10 + i, device=dev)
        gen = torch.Generator(device=dev).manual_seed(20 + i)
        with torch.no_grad():
            for t in mem.module.tables.values():
                t.weight.normal_(0.0, 1.0, generator=gen)
        h = wl.make_hidden(ws, seed=30 + i, device=dev)
        hn = ops.rmsnorm(h, torch.ones(ws.d_model, dtype=ws.dtype, device=dev), ws.norm_eps)
        pos = 2 * i
        if blocks:
            blocks.append(SimpleNamespace(memory=None))
        blocks.append(SimpleNamespace(memory=mem))
        inputs[pos] = (h, hn)
    return SimpleNamespace(blocks=blocks, tok_emb=None, ssm=None), inputs


def run(model, inputs, cuts, provider=None, st=None):
    """Decode the positions ``cuts[0] .. cuts[-1]`` in the blocks between cuts; outputs per layer."""
    b = next(iter(inputs.values()))[0].shape[0]
    st = st or DecodeState.empty(model, b, cuts[-1])
    outs = {p: [] for p in inputs}
    with torch.no_grad():
        for a, e in zip(cuts[:-1], cuts[1:]):
            for pos, (h, hn) in inputs.items():
                outs[pos].append(memory_decode(model, pos, st, h[:, a:e], h_norm=hn[:, a:e], row_provider=provider))
            st.length = e
    return {p: torch.cat(o, 1) for p, o in outs.items()}, st


def steps(prompt: int, total: int) -> list:
    return [0, prompt] + list(range(prompt + 1, total + 1))


# ------------------------------------------------------------------ layout
@pytest.mark.parametrize("variant", ["tiny", "sb"])
def test_serving_layout_route_tokens_candidates_and_involution(dev, variant):
    model, _ = make(variant, dev)
    m = model.blocks[0].memory.module
    R, bits = m.num_routes, m.bits_per_route
    tables = sl.permute_tables(m)
    for o, t in tables.items():
        back = sl.permute_table(t, R, o, bits)
        assert torch.equal(back, m.tables[f"ngram_{o}"].weight)
        rev = sl.reverse_digits(o, bits, dev)
        assert torch.equal(t.view(R, -1, t.shape[1]), m.tables[f"ngram_{o}"].weight.view(R, -1, t.shape[1])[:, rev])
    gen = torch.Generator(device=dev).manual_seed(3)
    codes = torch.randint(0, 16, (3, 20, R), device=dev, dtype=torch.uint8, generator=gen)
    with torch.no_grad():
        want = m._lookup_route_chunk(codes, None, 0, R, None, None)
    got = sl.serving_route_tokens(tables, codes, m.ngrams, bits)
    assert torch.equal(got, want)
    # the oracle's route tokens (lngram_v2.py:1047-1113) from the module's own tables, bit for bit
    otab = {o: m.tables[f"ngram_{o}"].weight.detach().cpu() for o in m.ngrams}
    assert torch.equal(got.cpu(), om.route_tokens(otab, codes.cpu().numpy(), m.ngrams, bits).to(got.dtype))
    # reverse_digits' known answers (reference tests/test_index_layout.py:40-43), and the serving
    # address = the oracle's aligned address (oldest code least significant) with its digits reversed
    r = sl.reverse_digits(3, 4, dev)
    assert torch.equal(r[r], torch.arange(4096, device=dev)) and int(r[1]) == 256 and int(r[16]) == 16
    for o in m.ngrams:
        addr = sl.serving_address(codes, o, bits)
        aligned = torch.from_numpy(om.ngram_address(codes.cpu().numpy(), o, bits)).to(dev)
        assert torch.equal(addr, sl.reverse_digits(o, bits, dev)[aligned])
    for t in range(2, 19):                                   # codes up to t known; rows of t + 1
        cands = sl.candidate_rows(tables, codes[:, t - 1:t + 1], m.ngrams, bits)
        for o, blk in cands.items():
            assert blk.shape == (3, R, 16, m.memory_dim)
            base = sl.candidate_base(codes[:, t - o + 2:t + 1], o, bits)
            assert torch.equal(blk, tables[o][base[..., None] + torch.arange(16, device=dev)])
        assert torch.equal(sl.select_candidates(cands, codes[:, t + 1], m.ngrams), want[:, t + 1])


def test_layer_table_index_paths_match_kernel_paths(dev):
    model, _ = make("tiny", dev)
    m = model.blocks[0].memory.module
    lt = LayerTable.from_module(m)
    assert lt.on_host and lt.weight.is_pinned()
    assert lt.nbytes == (m.num_routes * (16 ** 2 + 16 ** 3) + 1) * m.memory_dim * 4
    codes = torch.randint(0, 16, (2, 10, m.num_routes), device=dev, dtype=torch.uint8)
    with torch.no_grad():
        full = m._lookup_route_chunk(codes, None, 0, m.num_routes, None, None)
    for p in range(10):
        hist = codes[:, max(0, p - lt.history):p]
        cand = lt.gather(lt.candidate_index(hist, p))                      # [B, R, len, 16, D]
        assert torch.equal(cand, lt.candidates(hist, p))
        rows = cand.gather(3, codes[:, p].long()[:, :, None, None, None].expand(-1, -1, len(lt.ngrams), 1, lt.dim))
        assert torch.equal(rows[:, :, :, 0].flatten(2), full[:, p])
        ctx = codes[:, max(0, p - lt.history):p + 1]
        exact = lt.gather(lt.exact_index(ctx, 1))
        assert torch.equal(exact.flatten(3)[:, 0], full[:, p])
        assert torch.equal(lt.rows(ctx, 1)[:, 0], full[:, p])


# ------------------------------------------------------------------ B1 / B4
@pytest.mark.parametrize("variant", sorted(VARIANTS))
@pytest.mark.parametrize("threaded", [False, True])
def test_b1_b4_bitwise_equal_b0(dev, variant, threaded):
    model, inputs = make(variant, dev, seq=26)
    cuts = steps(5, 26)
    ref, _ = run(model, inputs, cuts)
    host = HostTables.from_model(model)
    offload_tables(model)
    b1 = HostGather(host, dev)
    b4 = CandidatePrefetcher(host, dev, threaded=threaded)
    try:
        for prov in (b1, b4):
            got, _ = run(model, inputs, cuts, prov)
            for p in ref:
                assert torch.equal(got[p], ref[p]), (variant, type(prov).__name__, p)
    finally:
        b4.close()
    s = b4.stats.summary()
    n_mem = len(host)
    # one prefill gather + 21 hits per layer; no stale history; no codes to the host
    assert s["hits"] == 21 * n_mem and s["misses"] == 0 and s["stale"] == 0
    assert s["tokens"] == 2 * 26 and s["d2h_bytes"] == 0


@pytest.mark.parametrize("plen", [1, 2])
def test_positions_0_and_1(dev, plen):
    model, inputs = make("sb", dev, seq=plen + 5)
    cuts = steps(plen, plen + 5)
    ref, _ = run(model, inputs, cuts)
    host = HostTables.from_model(model)
    offload_tables(model)
    b4 = CandidatePrefetcher(host, dev, threaded=False)
    got, _ = run(model, inputs, cuts, b4)
    assert torch.equal(got[0], ref[0])
    assert b4.stats.hits == 5


def test_rollback_and_new_state_are_misses_not_wrong(dev):
    model, inputs = make("tiny", dev, seq=20)
    (h, hn), = inputs.values()
    ref, _ = run(model, inputs, [0, 6] + list(range(7, 21)))
    host = HostTables.from_model(model)
    offload_tables(model)
    b4 = CandidatePrefetcher(host, dev)
    st = DecodeState.empty(model, 2, 20)
    got = []
    with torch.no_grad():
        memory_decode(model, 0, st, h[:, :6], h_norm=hn[:, :6], row_provider=b4)
        st.length = 6
        for t in range(6, 12):
            got.append(memory_decode(model, 0, st, h[:, t:t + 1], h_norm=hn[:, t:t + 1], row_provider=b4))
            st.length = t + 1
        st.truncate(9)                                   # the staged position (12) no longer matches
        for t in range(9, 20):
            got.append(memory_decode(model, 0, st, h[:, t:t + 1], h_norm=hn[:, t:t + 1], row_provider=b4))
            st.length = t + 1
        out = torch.cat(got[:3] + got[6:], 1)
        assert torch.equal(out, ref[0][:, 6:])
        assert b4.stats.misses == 1 and b4.stats.stale == 0
        # a new state object: its first single-token step is a miss as well
        st2 = DecodeState.empty(model, 2, 20)
        memory_decode(model, 0, st2, h[:, :4], h_norm=hn[:, :4], row_provider=b4)
        st2.length = 4
        o = memory_decode(model, 0, st2, h[:, 4:5], h_norm=hn[:, 4:5], row_provider=b4)
        assert torch.equal(o, ref[0][:, 4:5])
        assert b4.stats.hits == 17 and b4.stats.misses == 1
    b4.close()


def test_byte_accounting(dev):
    model, inputs = make("tiny", dev, seq=8)
    m = model.blocks[0].memory.module
    host = HostTables.from_model(model)
    cuts = [0, 4, 5, 6, 7, 8]
    b1, b4 = HostGather(host, dev), CandidatePrefetcher(host, dev, threaded=False)
    run(model, inputs, cuts, b1)
    run(model, inputs, cuts, b4)
    row = m.memory_dim * 4
    k = len(m.ngrams)

    def exact(n):
        return 2 * n * m.num_routes * k * row

    assert b1.stats.h2d_bytes == exact(4) + 4 * exact(1)
    cand = 2 * m.num_routes * k * 16 * row
    assert b4.stats.h2d_bytes == exact(4) + 5 * cand           # prefill gather + one candidate set per call
    assert b1.stats.summary()["h2d_bytes_per_token"] == b1.stats.h2d_bytes / 16
    b4.close()


def test_offload_restore_and_device_resident_tables(dev):
    model, inputs = make("sb", dev, seq=12)
    cuts = [0, 6, 9, 12]
    ref, _ = run(model, inputs, cuts)
    host = HostTables.from_model(model)
    dev_tables = HostTables.from_model(model, device=dev)           # the same movers over HBM
    assert offload_tables(model) > 0
    assert model.blocks[0].memory.module.tables["ngram_2"].weight.device.type == "meta"
    with pytest.raises(RuntimeError):
        run(model, inputs, cuts)                                     # no table, no provider: fails loudly
    got, _ = run(model, inputs, cuts, ZeroCopyGather(host, dev))
    assert torch.equal(got[0], ref[0])
    got, _ = run(model, inputs, cuts, HostGather(dev_tables, dev))
    assert torch.equal(got[0], ref[0])
    restore_tables(model, host)
    again, _ = run(model, inputs, cuts)
    assert torch.equal(again[0], ref[0])


# ------------------------------------------------------------------ verify blocks
def _codes_of(model, inputs, total):
    """The verifier's codes of every memory layer: a whole-block decode on the device."""
    _, st = run(model, inputs, [0, total])
    return {p: c[:, :total].clone() for p, c in st.codes.items()}


@pytest.mark.parametrize("bonus", ["all", "last"])
def test_staged_rows_equal_direct_lookup(dev, bonus):
    model, inputs = make("tiny_2mem", dev, seq=16)
    codes = _codes_of(model, inputs, 16)
    host = HostTables.from_model(model)
    stager = BlockStager(host, dev, bonus=bonus)
    for start, n in [(0, 3), (1, 4), (5, 5), (10, 5)]:
        blk = stager.stage(start, {p: c[:, start:start + n].cpu() for p, c in codes.items()},
                           {p: c[:, max(0, start - 2):start] for p, c in codes.items()})
        for pos, c in codes.items():
            m = model.blocks[pos].memory.module
            with torch.no_grad():
                full = m._lookup_route_chunk(c, None, 0, m.num_routes, None, None)
            assert torch.equal(blk.rows(pos), full[:, start:start + n])
            for j in range(n):
                if start + j + 1 >= 16:
                    continue
                br = blk.bonus_rows(pos, j, c[:, start + j + 1])
                if bonus == "last" and j < n - 1:
                    assert br is None
                else:
                    assert torch.equal(br, full[:, start + j + 1])
    stager.close()


@pytest.mark.parametrize("variant", ["tiny", "sb"])
def test_verify_blocks_equal_b0(dev, variant):
    model, inputs = make(variant, dev, seq=20)
    (h, hn), = inputs.values()
    codes = _codes_of(model, inputs, 20)
    ref, _ = run(model, inputs, [0, 6, 11, 20])
    host = HostTables.from_model(model)
    offload_tables(model)
    stager = BlockStager(host, dev)
    st = DecodeState.empty(model, 2, 20)

    def sl_(a, b):
        return ({p: c[:, a:b] for p, c in codes.items()}, {p: c[:, max(0, a - 2):a] for p, c in codes.items()})

    def step(a, b, prov):
        with torch.no_grad():
            o = memory_decode(model, 0, st, h[:, a:b], h_norm=hn[:, a:b], row_provider=prov)
        st.length = b
        return o

    out = [step(0, 6, stager.fallback)]
    blk = stager.stage(6, *sl_(6, 11))                         # verify block: positions 6..10
    out.append(step(6, 11, stager.provider(blk)))
    assert blk.codes_match()
    st.truncate(9)                                              # 2 drafts accepted after 6 -> bonus at 9
    nxt = stager.stage(10, *sl_(10, 14))                        # next drafts: positions 10..13
    out[-1] = out[-1][:, :3]
    out.append(step(9, 14, stager.provider(nxt, head=(blk, 2))))
    assert nxt.codes_match()
    out.append(step(14, 20, stager.provider(nxt)))               # wrong position -> fallback
    stager.close()
    got = torch.cat(out, 1)
    assert torch.equal(got, ref[0])
    assert stager.stats.hits == 2 and stager.stats.misses == 1
    # drafter codes that differ from the verifier's are reported
    st = DecodeState.empty(model, 2, 20)
    step(0, 6, stager.fallback)
    bad = {p: (c[:, 6:11] + 1) % 16 for p, c in codes.items()}
    blk2 = stager.stage(6, bad, {p: c[:, 4:6] for p, c in codes.items()})
    step(6, 11, stager.provider(blk2))
    assert not blk2.codes_match()


def test_staging_errors(dev):
    model, inputs = make("tiny", dev, seq=8)
    host = HostTables.from_model(model)
    with pytest.raises(ValueError, match="bonus"):
        BlockStager(host, dev, bonus="some")
    st = BlockStager(host, dev)
    codes = torch.zeros(2, 3, 8, dtype=torch.uint8)
    with pytest.raises(ValueError, match="history"):
        st.stage(4, {0: codes}, {0: codes[:, :1]})
    with pytest.raises(RuntimeError, match="CPU path"):
        HostGather(host, "cpu")
    st.close()
