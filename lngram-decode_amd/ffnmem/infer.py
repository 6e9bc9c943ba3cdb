"""Cached decoding of the memory layers: drop-in for the memory half of the reference
``ffnmem/infer.py`` (``DecodeState`` :65-112, ``ssm_continue`` :125-137, ``router_input_at``
:140-149, ``memory_step`` :152-182), for the memory part of ``static_verify``
(``drafting/live_spec.py:68-139``) and for the memory block of draft-tree verification
(``tree_verify_step``, ``drafting/tree.py:141-202``: ``tree_ssm_states``, ``tree_router_input``,
``tree_memory_step``).

The caches hold, per memory layer, the route codes of every processed position (uint8,
``[B, max_len, R]``) and the short conv's input rows (``[B, max_len, d]``), indexed by absolute
position, so rolling back is moving ``length``.  A step of ``n`` new positions runs the same
kernels as the whole-sequence forward, reading the cached history in place:

- the fused readout (``lng_memory_readout_fused_at``) takes each new token's n-gram rows from the
  code cache at positions ``t, t-1, t-2``; other shapes gather route tokens from the cached
  context (``lng_route_tokens``) and run the materialised readout;
- the short conv (``lng_causal_conv_at``) reads its causal window from the conv-input cache and
  normalises each row as the whole-sequence conv does.

So the cached outputs equal the full forward's up to the summation order of the projections
(identical where the same GEMM kernel serves both shapes).  ``conv_in`` differs from the
reference's in content, not in role: it keeps the conv's input rows before the conv's RMSNorm
(the reference keeps them after it); rows move the same way under ``truncate`` and tree
acceptance.

The attention and FFN halves of the reference's ``decode_step`` belong to the transformer, which
is not part of this path: ``DecodeState`` here caches the memory layers (``k`` / ``v`` stay empty).
A "model" is anything with ``blocks`` (each with a ``memory`` attribute, an ``LngramMemory`` or
None) and, for token-routed memories, ``tok_emb`` and ``ssm``; ``memory_model`` wraps a single
memory layer.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from types import SimpleNamespace

import torch
from torch import Tensor

from lngram_hip import ops


# ------------------------------------------------------------------ state
@dataclass
class DecodeState:
    batch: int
    max_len: int
    length: int = 0
    tokens: Tensor | None = None                       # [B, max_len]
    k: list = field(default_factory=list)              # attention caches: not on this path
    v: list = field(default_factory=list)
    codes: dict = field(default_factory=dict)          # block pos -> [B, max_len, R] uint8
    conv_in: dict = field(default_factory=dict)        # block pos -> [B, max_len, d] conv input rows
    ssm: Tensor | None = None                          # [B, max_len, N] fp32
    epoch: int = 0                                     # bumped on truncate

    @classmethod
    def empty(cls, model, batch: int, max_len: int, dtype: torch.dtype | None = None) -> "DecodeState":
        """``DecodeState.empty`` (``infer.py:78-97``) for the memory layers of ``model``."""
        s = cls(batch=batch, max_len=max_len)
        dev = None
        for pos, block in enumerate(model.blocks):
            mem = getattr(block, "memory", None)
            if mem is None:
                continue
            m = mem.module
            if m.execution_mode == "streaming":
                raise NotImplementedError("cached decoding with streaming memory readout")
            w = m.readout_o_proj.weight
            dev = w.device
            dt = dtype or w.dtype
            s.codes[pos] = torch.zeros(batch, max_len, mem.routes, dtype=torch.uint8, device=dev)
            s.conv_in[pos] = torch.zeros(batch, max_len, m.hidden_size, dtype=dt, device=dev)
        if dev is None:
            raise ValueError("the model has no memory layer")
        s.tokens = torch.zeros(batch, max_len, dtype=torch.long, device=dev)
        ssm = getattr(model, "ssm", None)
        if ssm is not None:
            s.ssm = torch.zeros(batch, max_len, ssm.state_dim, dtype=torch.float32, device=dev)
        return s

    def truncate(self, length: int) -> None:
        if not 0 <= length <= self.length:
            raise ValueError(f"cannot truncate to {length} (length {self.length})")
        self.length = length
        self.epoch += 1

    def index_select(self, idx: Tensor) -> "DecodeState":
        """Rows ``idx`` of every cache (``infer.py:105-111``)."""
        def sel(t):
            return t.index_select(0, idx.to(t.device))

        return DecodeState(len(idx), self.max_len, self.length, sel(self.tokens), [], [],
                           {p: sel(t) for p, t in self.codes.items()},
                           {p: sel(t) for p, t in self.conv_in.items()},
                           None if self.ssm is None else sel(self.ssm), self.epoch)


def memory_model(mem, tok_emb=None, ssm=None):
    """A one-block "model" around an ``LngramMemory`` for the functions below (block 0)."""
    return SimpleNamespace(blocks=[SimpleNamespace(memory=mem)], tok_emb=tok_emb, ssm=ssm)


# ------------------------------------------------------------------ pieces
def ssm_continue(model, emb: Tensor, s_prev: Tensor | None) -> Tensor:
    """SSM states of new positions from the state before them (``infer.py:125-137``):
    ``lng_ssm_scan`` with the carried state as ``s0``."""
    ssm = model.ssm
    return ops.ssm_scan(ssm.decay(), ssm.inputs(emb), s_prev)


def router_input_at(model, mem, state: DecodeState, emb: Tensor, s_new: Tensor | None) -> Tensor:
    """Token-only router features of the new positions (``infer.py:140-149``): the previous
    token's embedding comes from the cache."""
    L = state.length
    if L == 0:
        return mem.router_features(emb, s_new)
    prev = model.tok_emb(state.tokens[:, L - 1:L]).to(emb.dtype)
    s_cat = None
    if s_new is not None:
        s_cat = torch.cat((state.ssm[:, L - 1:L], s_new), dim=1)
    return mem.router_features(torch.cat((prev, emb), dim=1), s_cat)[:, 1:]


def _readout_head(m, h: Tensor, codes: Tensor, pos0: int, pos0_dev: Tensor | None) -> Tensor:
    """Fused readout of the new positions whose codes sit at ``pos0 (+ pos0_dev)`` of ``codes``."""
    q_raw = ops.linear(h, m._folded_query_weight())
    return ops.memory_readout_fused_at(q_raw, codes, pos0, m.tables["ngram_2"].weight, m.tables["ngram_3"].weight,
                                       m._fused_weights(), m.readout_memory_norm.weight, m.readout_memory_norm.eps,
                                       m.softmax_scale, m.readout_sink_logit, q_rows=h,
                                       q_eps=m.readout_query_norm.eps, pos0_dev=pos0_dev)


def _skinny_ok(x: Tensor, w: Tensor) -> bool:
    """Whether ``lng_linear_at`` / ``lng_router_codes_at`` take ``x [B, n, K] . w^T`` (the decode
    projections written straight into a cache)."""
    return (x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and x.shape[0] * x.shape[1] <= 64
            and x.shape[-1] % 32 == 0 and w.shape[0] % 16 == 0)


def _oproj_to_cache(m, head: Tensor, conv_in: Tensor, L: int, n: int, L_dev: Tensor | None) -> None:
    """``mixed = W_o head``, cached as conv input at positions L .. L+n-1 (+ L_dev)."""
    b = head.shape[0]
    x = head.reshape(b, n, m.readout_inner_dim)
    w_o = m.readout_o_proj.weight
    conv = m.short_conv
    if conv.conv.bias is not None:
        raise NotImplementedError("conv bias is not supported by lng_causal_conv")
    if _skinny_ok(x, w_o) and conv_in.dtype == torch.bfloat16:
        ops.linear_at(x, w_o, conv_in, L, L_dev)     # the projection writes the cache rows
    else:
        mixed = ops.linear(x, w_o)
        conv._check(mixed, None)
        if L_dev is None:
            conv_in[:, L:L + n] = mixed
        else:
            conv_in.index_copy_(1, L_dev.long() + torch.arange(n, device=x.device), mixed.to(conv_in.dtype))


def _finish_cached(m, head: Tensor, conv_in: Tensor, L: int, n: int, L_dev: Tensor | None) -> Tensor:
    """``mixed = W_o head``, cached as conv input at positions L .. L+n-1 (+ L_dev), then
    ``mixed + short_conv`` over the cached window (``infer.py:175-182``)."""
    _oproj_to_cache(m, head, conv_in, L, n, L_dev)
    conv = m.short_conv
    length = L + n if L_dev is None else conv_in.shape[1]
    return ops.causal_conv_at(conv_in, conv.norm.weight, conv.conv.weight, conv.dilation, conv.norm.eps,
                              pos0=L, n=n, length=length, pos0_dev=L_dev, residual=True)


def memory_step(model, pos: int, state: DecodeState, h: Tensor, codes_new: Tensor,
                route_codes_ctx: Tensor | None = None, route_tokens: Tensor | None = None) -> Tensor:
    """Memory output ``[B, n, d]`` of the new positions (``infer.py:152-182``); ``codes_new``
    ``[B, n, R]`` are written into the cache.  ``route_codes_ctx [B, n + H, R]`` replaces the
    cached codes for the lookup only (the n-grams ending at the new positions are read from it);
    as in the reference, the short conv still reads the cached rows in position order.  A draft
    tree's verification, whose windows and conv follow each node's ancestors
    (``tree.py:179-196``), is :func:`tree_memory_step`'s.  ``route_tokens [B, n, R, len(ngrams) * mem_dim]`` are rows supplied by
    the caller (the gather is skipped)."""
    mem = model.blocks[pos].memory
    m = mem.module
    L, n = state.length, h.shape[1]
    if L + n > state.max_len:
        raise ValueError(f"cache full: {L} + {n} > {state.max_len}")
    cache = state.codes[pos]
    cache[:, L:L + n] = codes_new.to(cache.dtype)
    if route_tokens is not None and m._fused_shape_ok(h, tables=False):
        # rows from the caller (host-RAM serving, staged verify blocks): the same fused readout
        q_raw = ops.linear(h, m._folded_query_weight())
        head = ops.memory_readout_fused_rows(q_raw, route_tokens.to(h.device, torch.bfloat16), m._fused_weights(),
                                             m.readout_memory_norm.weight, m.readout_memory_norm.eps, m.softmax_scale,
                                             m.readout_sink_logit, q_rows=h, q_eps=m.readout_query_norm.eps)
    elif route_tokens is None and m._fused_shape_ok(h):
        if route_codes_ctx is None:
            head = _readout_head(m, h, cache, L, None)
        else:
            ctx = route_codes_ctx.to(torch.uint8).contiguous()
            head = _readout_head(m, h, ctx, ctx.shape[1] - n, None)
    else:
        if route_tokens is None:
            ctx = route_codes_ctx
            if ctx is None:
                ctx = cache[:, max(0, L - m.route_history_length):L + n]
            tokens = m._lookup_route_chunk(ctx, None, 0, m.num_routes, None, None, target_length=n)
        else:
            tokens = route_tokens.to(h.device, m.readout_kv_proj.weight.dtype)
        key, value = m._project_memory(tokens)
        head = m._manual_gqa(m._project_query(h), key, value)
    return _finish_cached(m, head, state.conv_in[pos], L, n, None)


def static_memory_step(model, pos: int, state: DecodeState, h: Tensor, codes_new: Tensor | None, L_t: Tensor,
                       router_x: Tensor | None = None) -> Tensor:
    """``memory_step`` with shapes independent of the cached length (the memory part of
    ``static_verify``, ``live_spec.py:100-114``): ``L_t`` is a 0-d device tensor holding the
    length (int32 saves a conversion), the kernels read it on the device and write the caches at
    ``L_t .. L_t+n-1`` themselves (bf16, B*n <= 64; else ``index_copy_``), so the launches can be
    captured in a HIP graph and replayed for any length.  ``codes_new`` None: the codes are
    computed from ``router_x`` (``h_norm`` or the token features) straight into the code cache.
    The caller advances ``state.length`` (and ``L_t``) afterwards."""
    mem = model.blocks[pos].memory
    m = mem.module
    n = h.shape[1]
    dev = h.device
    L32 = (L_t if L_t.dtype == torch.int32 else L_t.to(torch.int32)).reshape(1)
    cache = state.codes[pos]
    if codes_new is None:
        if router_x is None:
            raise ValueError("static_memory_step needs codes_new or router_x")
        if _skinny_ok(router_x, mem.router.weight) and mem.bits == 4:
            ops.router_codes_at(router_x, mem.router.weight, cache, 0, L32)
        else:
            codes_new = mem.route_codes(router_x)[1]
    if codes_new is not None:
        cache.index_copy_(1, L32.long() + torch.arange(n, device=dev), codes_new.to(cache.dtype))
    if m._fused_shape_ok(h):
        head = _readout_head(m, h, cache, 0, L32)
    else:
        hist = m.route_history_length
        hidx = L32.long() - hist + torch.arange(hist + n, device=dev)
        ctx = cache.index_select(1, hidx.clamp_min(0))
        seg = (hidx >= 0).to(torch.int32)
        tokens = m._lookup_route_chunk(ctx, None, 0, m.num_routes, seg[None].expand(h.shape[0], -1).contiguous(),
                                       None, target_length=n)
        key, value = m._project_memory(tokens)
        head = m._manual_gqa(m._project_query(h), key, value)
    return _finish_cached(m, head, state.conv_in[pos], 0, n, L32)


def memory_decode(model, pos: int, state: DecodeState, h: Tensor, h_norm: Tensor | None = None,
                  router_in: Tensor | None = None, route_codes_ctx: Tensor | None = None, row_provider=None) -> Tensor:
    """The memory block of the reference's ``decode_step`` (``infer.py:226-241``): the new positions'
    route codes, then ``row_provider(pos, state, codes) -> route tokens [B, n, R, len*D] | None``
    (host-RAM serving; called before the codes enter the cache, ``state.length`` still L), then
    ``memory_step``.  The caller advances ``state.length`` after the step, as ``decode_step`` does."""
    codes = memory_codes(model, pos, state, h_norm=h_norm, router_in=router_in)
    rows = None if row_provider is None else row_provider(pos, state, codes)
    return memory_step(model, pos, state, h, codes, route_codes_ctx, rows)


# ------------------------------------------------------------------ draft-tree verification
def tree_ssm_states(model, state: DecodeState, emb: Tensor, parent) -> Tensor:
    """SSM states of the tree nodes ``emb [B, n, d]`` after the cached positions
    (``tree_verify_step``, ``drafting/tree.py:153-161``): each node continues from its parent's
    state, the root from the cached state at ``L - 1`` (zero at ``L = 0``); ``lng_ssm_tree``.
    The caller writes them into ``state.ssm`` after the step, as the reference does."""
    ssm = model.ssm
    L = state.length
    root = state.ssm[:, L - 1] if L > 0 else None
    return ops.ssm_tree(ssm.decay(), ssm.inputs(emb), _parent_index(parent, emb.device)[0], root)


def tree_router_input(model, mem, state: DecodeState, emb: Tensor, s_new: Tensor | None, parent) -> Tensor:
    """Token-router features of the tree nodes (``drafting/tree.py:170-177``): each node's previous
    token is its parent's; the root's is the last cached token (``start`` at ``L = 0``)."""
    feats = mem.router_features
    b, n, d = emb.shape
    L = state.length
    if L > 0:
        root_prev = model.tok_emb(state.tokens[:, L - 1]).to(emb.dtype)
    else:
        root_prev = feats.start.to(emb.dtype).expand(b, d)
    src = _parent_index(parent, emb.device)[1]          # node i's previous row: 0 the root's, p + 1 node p
    prev = torch.cat((root_prev[:, None], emb), 1).index_select(1, src)
    return feats.step(prev, emb, s_new)


_TREE_INDEX: dict = {}


def _parent_index(parent, device) -> tuple:
    """``(parent int32 [n], parent + 1 int64 [n])`` on the device, built once per tree shape."""
    key = ("parent", tuple(int(p) for p in parent), str(device))
    t = _TREE_INDEX.get(key)
    if t is None:
        par = torch.as_tensor(key[1], dtype=torch.int32)
        t = (par.to(device), (par.to(torch.long) + 1).clamp_min(0).to(device))
        _TREE_INDEX[key] = t
    return t


def _tree_index(parent, hist: int, back: int, device) -> tuple:
    """Device index tables of a tree shape, built once per (parent, hist, back, device):
    ``idx [n, hist + 1]``, the n-gram window slots of every node in ``cat(history of hist codes,
    node codes)`` (``tree_slots`` with a history of ``hist`` positions), ``rel [n, back + 1]``
    int32, the conv window slots relative to the cached length (negative: history positions), and
    ``idx`` as int32."""
    from drafting.tree import tree_slots

    key = (tuple(int(p) for p in parent), int(hist), int(back), str(device))
    t = _TREE_INDEX.get(key)
    if t is None:
        idx, _ = tree_slots(parent, hist, hist)          # every slot lies in the window's reach
        full, _ = tree_slots(parent, back + 1, back)     # all valid at a length of back + 1
        t = (idx.to(device), (full - (back + 1)).to(torch.int32).to(device), idx.to(torch.int32).to(device))
        _TREE_INDEX[key] = t
    return t


def _tree_memory(model, pos: int, state: DecodeState, h: Tensor, codes: Tensor, parent, L: int,
                 L_t: Tensor | None) -> Tensor:
    """``tree_memory_step`` at the cached length ``L`` (host) or ``*L_t`` (device int32, L = 0)."""
    mem = model.blocks[pos].memory
    m = mem.module
    b, n = h.shape[0], h.shape[1]
    dev = h.device
    if len(parent) != n:
        raise ValueError(f"tree_memory_step: {len(parent)} parents for {n} nodes")
    cache = state.codes[pos]
    hist = m.route_history_length
    conv = m.short_conv
    _, rel, idx32 = _tree_index(parent, hist, conv.left_padding, dev)
    r = cache.shape[-1]
    L_dev = None if L_t is None else L_t.to(torch.int32).reshape(1)
    # the node windows over (the last `hist` cached codes, the nodes' codes; a history slot before
    # position 0 is not real and its n-grams read zero rows), the node codes cached at L .. L+n-1 and
    # the conv slots, in one launch (the code caches are uint8: codes have at most 8 bits)
    win, seg, val, slots = ops.tree_windows(cache, codes, idx32, hist, L, L_dev, rel)
    tables = [m.tables[f"ngram_{o}"].weight for o in m.ngrams]
    rt = ops.route_tokens(win, tables, m.ngrams, m.bits_per_route, 0, m.num_routes, seg, val, 1)
    rt = rt[:, -1].view(b, n, r, -1)
    if m._fused_shape_ok(h, tables=False):
        q_raw = ops.linear(h, m._folded_query_weight())
        head = ops.memory_readout_fused_rows(q_raw, rt.to(torch.bfloat16), m._fused_weights(),
                                             m.readout_memory_norm.weight, m.readout_memory_norm.eps, m.softmax_scale,
                                             m.readout_sink_logit, q_rows=h, q_eps=m.readout_query_norm.eps)
    else:
        key, value = m._project_memory(rt.to(m.readout_kv_proj.weight.dtype))
        head = m._manual_gqa(m._project_query(h), key, value)
    conv_in = state.conv_in[pos]
    _oproj_to_cache(m, head, conv_in, L, n, L_dev)
    length = L + n if L_t is None else conv_in.shape[1]
    return ops.causal_conv_slots(conv_in, conv.norm.weight, conv.conv.weight, conv.dilation, conv.norm.eps, slots,
                                 length=length, residual=True)


def tree_memory_step(model, pos: int, state: DecodeState, h: Tensor, codes: Tensor, parent) -> Tensor:
    """The memory block of the reference's draft-tree verification (``tree_verify_step``,
    ``drafting/tree.py:179-196``) for the tree nodes ``h [B, n, d]`` after the ``L = state.length``
    cached positions.  Each node's n-gram windows follow its ancestors, then the cached history
    (``tree_ngram_codes`` / ``tree_route_tokens``); the readout runs over those rows; the output
    projection's rows go into the conv-input cache at ``L .. L+n-1`` in node order and the short
    conv reads each node's ancestor window of them (``tree_slots``, ``lng_causal_conv_slots``).
    ``codes [B, n, R]`` are the nodes' route codes (``memory_codes`` over their router inputs) and
    are cached at ``L .. L+n-1`` too.  Returns ``mixed + short_conv`` ``[B, n, d]``; the caller sets
    ``state.length`` (after the accepted path is compacted, as the reference's loop does).  Node i's
    output equals ``memory_step``'s for the last token of a chain decode along its root path."""
    L, n = state.length, h.shape[1]
    if L + n > state.max_len:
        raise ValueError(f"cache full: {L} + {n} > {state.max_len}")
    return _tree_memory(model, pos, state, h, codes, parent, L, None)


def static_tree_memory_step(model, pos: int, state: DecodeState, h: Tensor, codes: Tensor, parent,
                            L_t: Tensor) -> Tensor:
    """``tree_memory_step`` with the cached length in ``L_t`` (a 0-d device int32): no host
    synchronisation and shapes independent of the length, so the launches can be captured in a HIP
    graph and replayed at any length (the tree verification of ``static_verify``-style loops).  The
    caller keeps ``L_t + n <= state.max_len``; the device length is not checked on the host."""
    return _tree_memory(model, pos, state, h, codes, parent, 0, L_t)


# ------------------------------------------------------------------ one memory layer's step
def memory_codes(model, pos: int, state: DecodeState, h_norm: Tensor | None = None,
                 router_in: Tensor | None = None) -> Tensor:
    """Route codes of the new positions (``infer.py:230-236``): the router reads ``h_norm``
    (hidden router) or the token features ``router_in``."""
    mem = model.blocks[pos].memory
    x = h_norm if mem.router_input == "hidden" else router_in
    if x is None:
        raise ValueError(f"router_input={mem.router_input} needs {'h_norm' if mem.router_input == 'hidden' else 'router_in'}")
    return mem.route_codes(x)[1]
