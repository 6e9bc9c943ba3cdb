"""Oracle: CPU restatement of the route n-gram memory forward (test infrastructure only).

Integer work (codes, addresses, rows) is numpy; floating-point work is torch on the
CPU in the op order of the reference, parameterised by dtype:

- ``torch.float64``  : a high-precision restatement (the tight oracle);
- ``torch.float32``  : the reference's fp32 path;
- ``torch.bfloat16`` : the reference's bf16 path (``load_model(dtype=bfloat16)``
  semantics: every module op in bf16 with its own rounding, the router in fp32).

Every function cites the reference lines it restates.  Parameters are passed as a
plain dict keyed like the reference module's ``state_dict`` (``tables.ngram_2.weight``,
``readout_q_proj.weight``, ... and ``router.weight`` for the wrapper).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch
import torch.nn.functional as F


# ----------------------------------------------------------------------------- config
@dataclass(frozen=True)
class MemCfg:
    """Shape of one memory layer (reference: ``wrapper.py:50-95`` + ``lngram_v2.py:842-1010``)."""

    d_model: int
    routes: int
    mem_dim: int
    q_heads: int
    kv_heads: int
    head_dim: int
    bits: int = 4
    orders: tuple = (2, 3)
    eps: float = 1e-5
    conv_kernel: int = 4
    sink_mass: float = 0.5

    @property
    def route_token_dim(self) -> int:
        return len(self.orders) * self.mem_dim

    @property
    def groups(self) -> int:
        return self.q_heads // self.kv_heads

    @property
    def conv_dilation(self) -> int:
        # lngram_v2.py:1000-1010 -- dilation defaults to the largest n-gram order
        return max(self.orders)

    @property
    def sink_logit(self) -> float:
        # lngram_v2.py:1877-1885 -- b0 = log(R (1 - m) / m)
        return math.log(self.routes * (1.0 - self.sink_mass) / self.sink_mass)

    @property
    def softmax_scale(self) -> float:
        return self.head_dim ** -0.5


# ----------------------------------------------------------------------------- integer parts
def pack_route_codes(logits, bits: int) -> np.ndarray:
    """Route codes from router logits.

    Follows ``lngram_v2.py:1012-1017`` (``q_logits > 0``) and ``:74-89``
    (bit i of route r is channel ``r*bits + i``; code = sum bit_i << i).  Strict ``>``:
    0, -0 and NaN give bit 0.  Returns int32 ``[..., R]``.
    """
    q = np.asarray(logits)
    *lead, c = q.shape
    if c % bits:
        raise ValueError("channels must be divisible by bits")
    b = (q > 0).reshape(*lead, c // bits, bits).astype(np.int32)
    return (b << np.arange(bits, dtype=np.int32)).sum(-1).astype(np.int32)


def ngram_address(codes, order: int, bits: int) -> np.ndarray:
    """``_aligned_ngram_address`` (``lngram_v2.py:314-325``).

    ``addr[b, t', r] = sum_k codes[b, t'+k, r] << (k*bits)`` for ``t' = 0 .. T-order``:
    the oldest code of the window is the least significant digit.
    """
    c = np.asarray(codes).astype(np.int64)
    b, t, r = c.shape
    n_valid = t - order + 1
    if n_valid <= 0:
        return np.zeros((b, 0, r), np.int64)
    out = np.zeros((b, n_valid, r), np.int64)
    for k in range(order):
        out |= c[:, k:k + n_valid] << (k * bits)
    return out


def valid_mask(order: int, batch: int, time: int, segment_ids=None, valid_tokens=None) -> np.ndarray:
    """``_valid_mask`` (``lngram_v2.py:1027-1045``): position t has an order-n row iff
    ``t >= n-1`` and the window's first and last positions share a segment (and the
    last position is a valid token)."""
    v = np.zeros((batch, time), bool)
    if time < order:
        return v
    s = np.ones((batch, time - order + 1), bool)
    if segment_ids is not None:
        seg = np.asarray(segment_ids)
        s &= seg[:, : time - order + 1] == seg[:, order - 1:]
    if valid_tokens is not None:
        s &= np.asarray(valid_tokens, bool)[:, order - 1:]
    v[:, order - 1:] = s
    return v


def route_rows(codes, orders, bits: int, route_start: int = 0, route_end: int | None = None,
               segment_ids=None, valid_tokens=None) -> np.ndarray:
    """Global table rows read by ``_lookup_route_chunk`` (``lngram_v2.py:1047-1092``).

    Returns int64 ``[B, T, route_end-route_start, len(orders)]``; ``row = r * 2^(bits*n)
    + addr`` (``:1064-1084``) and ``-1`` where the reference multiplies the row by a
    zero validity mask (``:1085-1092``).
    """
    c = np.asarray(codes).astype(np.int64)
    b, t, r_all = c.shape
    route_end = r_all if route_end is None else route_end
    rr = np.arange(route_start, route_end, dtype=np.int64)
    out = np.full((b, t, route_end - route_start, len(orders)), -1, np.int64)
    for oi, n in enumerate(orders):
        vm = valid_mask(n, b, t, segment_ids, valid_tokens)
        addr = ngram_address(c[:, :, route_start:route_end], n, bits)
        if addr.shape[1] == 0:
            continue
        rows = rr[None, None, :] * (1 << (bits * n)) + addr
        blk = out[:, n - 1:, :, oi]
        blk[...] = rows
        out[..., oi] = np.where(vm[..., None], out[..., oi], -1)
    return out


def route_tokens(tables: dict, codes, orders, bits: int, route_start: int = 0, route_end: int | None = None,
                 segment_ids=None, valid_tokens=None, target_length: int | None = None) -> torch.Tensor:
    """Route tokens ``[B, T, R', len(orders)*mem_dim]`` (``lngram_v2.py:1047-1113``):
    per order the gathered row (zero where invalid), concatenated over orders in the
    feature dimension (2-gram first), optionally the last ``target_length`` positions."""
    rows = route_rows(codes, orders, bits, route_start, route_end, segment_ids, valid_tokens)
    parts = []
    for oi, n in enumerate(orders):
        tab = tables[n]
        sel = torch.from_numpy(rows[..., oi])
        got = tab[sel.clamp_min(0)]
        parts.append(got * (sel >= 0).unsqueeze(-1).to(got.dtype))
    out = torch.cat(parts, -1)
    if target_length is not None:
        out = out[:, -int(target_length):]
    return out


def mix32(h) -> np.ndarray:
    """MurmurHash3's 32-bit finaliser ``fmix32`` (Appleby, MurmurHash3.cpp, public domain) in uint32
    arithmetic: ``h ^= h >> 16; h *= 0x85ebca6b; h ^= h >> 13; h *= 0xc2b2ae35; h ^= h >> 16``.
    Not from the reference: it defines the slot choice of the scaled-table workload."""
    h = np.asarray(h, dtype=np.uint64) & 0xFFFFFFFF
    h ^= h >> 16
    h = (h * 0x85EBCA6B) & 0xFFFFFFFF
    h ^= h >> 13
    h = (h * 0xC2B2AE35) & 0xFFFFFFFF
    h ^= h >> 16
    return h


def scaled_rows(codes, orders, bits: int, scale_log2: int, seed: int) -> np.ndarray:
    """Rows read from tables grown ``S = 2**scale_log2`` times per route (the scaled-table
    configuration: ``serving/scaled_tables.py:1-22`` grows the table, here at a fixed route count).

    int64 ``[B, T, R, len(orders)]``: ``row = (r*S + slot) * 2^(bits n) + addr_n``, -1 where
    ``route_rows`` (``lngram_v2.py:1047-1092``) masks the row (t < n-1).  ``addr_n`` is the
    reference's aligned address of the codes masked to ``bits``; ``slot = mix32(seed ^
    mix32(p * 0x9E3779B1 + r * n_orders + i)) & (S-1)`` with ``p = b*T + t`` and ``i`` the order's
    index.  With ``scale_log2 = 0`` the rows are the reference's global rows."""
    c = np.asarray(codes).astype(np.int64) & ((1 << bits) - 1)
    b, t, r = c.shape
    base = route_rows(c, orders, bits)                        # r * 2^(bits n) + addr, or -1
    S = 1 << scale_log2
    p = np.arange(b * t, dtype=np.uint64).reshape(b, t, 1, 1)
    i = (np.arange(r, dtype=np.uint64)[:, None] * len(orders) + np.arange(len(orders), dtype=np.uint64)[None, :])
    slot = (mix32(np.uint64(seed & 0xFFFFFFFF) ^ mix32((p * 0x9E3779B1 + i[None, None]) & 0xFFFFFFFF))
            & np.uint64(S - 1)).astype(np.int64)
    blk = np.array([1 << (bits * n) for n in orders], np.int64)
    rr = np.arange(r, dtype=np.int64)[:, None]
    rows = base + (rr * (S - 1) + slot) * blk                 # (r S + slot) 2^(bits n) + addr
    return np.where(base >= 0, rows, -1)


def gather_sum_scaled(tables, codes, orders, bits: int, scale_log2: int, seed: int,
                      positions=None) -> np.ndarray:
    """fp64 ``[B, T, mem_dim]`` (or ``[len(positions), mem_dim]`` for flat token indices
    ``positions``): the sum over routes and orders of the rows of ``scaled_rows`` (a masked row
    adds nothing).  ``tables`` are torch tensors (any device) indexed by the computed rows."""
    rows = scaled_rows(codes, orders, bits, scale_log2, seed)
    b, t, r, no = rows.shape
    flat = rows.reshape(b * t, r, no)
    if positions is not None:
        flat = flat[np.asarray(positions)]
    md = tables[0].shape[1]
    out = np.zeros((flat.shape[0], md), np.float64)
    for oi in range(no):
        sel = flat[:, :, oi]
        ok = sel >= 0
        idx = torch.from_numpy(np.where(ok, sel, 0).reshape(-1)).to(tables[oi].device)
        got = tables[oi][idx].double().cpu().numpy().reshape(flat.shape[0], r, md)
        out += (got * ok[..., None]).sum(1)
    return out if positions is not None else out.reshape(b, t, md)


def gather_sum_rows_torch(tables, rows: np.ndarray) -> torch.Tensor:
    """The gather of ``_lookup_route_chunk`` (``lngram_v2.py:1084-1092``: embedding lookup in the
    table dtype, masked rows multiplied by 0) followed by an fp32 sum over routes and orders, in
    PyTorch on the tables' device: fp32 ``[B, T, mem_dim]`` from int64 rows ``[B, T, R, n_orders]``
    (-1 = masked).  The CPU-timed form of ``gather_sum_scaled``; the tests hold it to that fp64
    restatement."""
    b, t, r, no = rows.shape
    out = torch.zeros(b * t, tables[0].shape[1], dtype=torch.float32)
    for oi in range(no):
        sel = torch.from_numpy(rows[..., oi].reshape(b * t, r))
        ok = sel >= 0
        got = torch.nn.functional.embedding(sel.clamp_min(0), tables[oi]) * ok[..., None].to(tables[oi].dtype)
        out += got.float().sum(1)
    return out.reshape(b, t, -1)


# ----------------------------------------------------------------------------- float parts
def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """``model.RMSNorm`` (``model.py:39-48``), the norm of ``h_norm`` and of the token router
    features: normalise in fp32 (fp64 for fp64 input), round to the input dtype, then multiply
    by the weight in that dtype (two roundings for bf16)."""
    work = torch.float64 if x.dtype == torch.float64 else torch.float32
    xf = x.to(work)
    y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return y.to(x.dtype) * w.to(x.dtype)


def rms_norm_v2(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """``lngram_v2.RMSNorm`` (``lngram_v2.py:36-53``), the memory module's query, memory and
    short-conv norms: ``F.rms_norm``, which normalises and applies the weight in fp32 and rounds
    once to the input dtype (fp64 stays fp64)."""
    work = torch.float64 if x.dtype == torch.float64 else torch.float32
    xf = x.to(work)
    y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * w.to(x.dtype).to(work)
    return y.to(x.dtype)


def rms_norm_fp32(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """``cpu_drafter._rms`` (``drafting/cpu_drafter.py:64-65``): everything in x's dtype."""
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def sink_probabilities(scores: torch.Tensor, sink_logit: float) -> torch.Tensor:
    """``_real_route_probabilities`` (``lngram_v2.py:1887-1897``): softmax over routes
    with one extra zero-value logit ``b0`` in the denominator, in fp32 (fp64 stays fp64)."""
    s = scores if scores.dtype == torch.float64 else scores.float()
    sink = torch.tensor(sink_logit, dtype=s.dtype)
    m = torch.maximum(s.amax(-1, keepdim=True), sink)
    ex = torch.exp(s - m)
    return ex / (ex.sum(-1, keepdim=True) + torch.exp(sink - m))


def _p(params: dict, key: str, dtype) -> torch.Tensor:
    return params[key].to(dtype)


def project_query(params: dict, cfg: MemCfg, h: torch.Tensor) -> torch.Tensor:
    """``_project_query`` (``lngram_v2.py:1115-1118``): ``W_q RMSNorm(h)`` -> [B, T, H, hd]."""
    dt = h.dtype
    x = rms_norm_v2(h, _p(params, "readout_query_norm.weight", dt), cfg.eps)
    q = F.linear(x, _p(params, "readout_q_proj.weight", dt))
    return q.view(*h.shape[:-1], cfg.q_heads, cfg.head_dim)


def project_memory(params: dict, cfg: MemCfg, tokens: torch.Tensor):
    """``_project_memory`` (``lngram_v2.py:1120-1131``): memory RMSNorm over Dt, KV
    projection, split keys first, reshape to ``[B, T, KV, R, hd]`` each."""
    dt = tokens.dtype
    x = rms_norm_v2(tokens, _p(params, "readout_memory_norm.weight", dt), cfg.eps)
    kv = F.linear(x, _p(params, "readout_kv_proj.weight", dt))
    kh = cfg.kv_heads * cfg.head_dim
    key, value = kv[..., :kh], kv[..., kh:]
    b, t, r, _ = key.shape
    key = key.reshape(b, t, r, cfg.kv_heads, cfg.head_dim).permute(0, 1, 3, 2, 4)
    value = value.reshape(b, t, r, cfg.kv_heads, cfg.head_dim).permute(0, 1, 3, 2, 4)
    return key, value


def manual_gqa(cfg: MemCfg, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor) -> torch.Tensor:
    """v2 ``_manual_gqa`` (``lngram_v2.py:1899-1920``): query heads grouped as
    ``[KV, G]`` (head = kv*G + g); scores = (q . k) in the storage dtype, then fp32 times
    ``hd^-0.5``; sink softmax; ``p.to(v.dtype) @ v``."""
    b, t = query.shape[:2]
    g = query.reshape(b, t, cfg.kv_heads, cfg.groups, cfg.head_dim)
    scores = torch.matmul(g, key.transpose(-1, -2).contiguous())
    scores = (scores if scores.dtype == torch.float64 else scores.float()) * cfg.softmax_scale
    p = sink_probabilities(scores, cfg.sink_logit)
    out = torch.matmul(p.to(value.dtype), value)
    return out.reshape(b, t, cfg.q_heads, cfg.head_dim)


def causal_conv(params: dict, cfg: MemCfg, mixed: torch.Tensor, segment_ids=None) -> torch.Tensor:
    """``DepthwiseCausalConv.forward`` (``lngram_v2.py:273-286``, ``:244-271`` for
    segments): ``SiLU(conv(RMSNorm(mixed)))`` with kernel K, dilation = max order, zero
    left padding ``(K-1)*dil``, no bias.  Tap j reads lag ``(K-1-j)*dil`` (Conv1d stores
    taps oldest -> newest)."""
    dt = mixed.dtype
    x = rms_norm_v2(mixed, _p(params, "short_conv.norm.weight", dt), cfg.eps)
    w = _p(params, "short_conv.conv.weight", dt)  # [d, 1, K]
    k, dil = cfg.conv_kernel, cfg.conv_dilation
    if segment_ids is None:
        xin = F.pad(x.transpose(1, 2), ((k - 1) * dil, 0))
        y = F.conv1d(xin, w, None, 1, 0, dil, x.shape[-1]).transpose(1, 2)
        return F.silu(y)
    seg = torch.as_tensor(np.asarray(segment_ids))
    out = torch.zeros_like(x)
    b, t, c = x.shape
    for tap in range(k):
        lag = (k - 1 - tap) * dil
        if lag == 0:
            sh, ok = x, torch.ones(b, t, 1, dtype=torch.bool)
        else:
            sh = F.pad(x[:, :-lag], (0, 0, lag, 0)) if lag < t else torch.zeros_like(x)
            ok = torch.zeros(b, t, 1, dtype=torch.bool)
            if lag < t:
                ok[:, lag:, 0] = seg[:, lag:] == seg[:, :-lag]
        out = out + sh * ok.to(sh.dtype) * w[:, 0, tap].view(1, 1, c)
    return F.silu(out)


def finish(params: dict, cfg: MemCfg, head: torch.Tensor, segment_ids=None) -> torch.Tensor:
    """``_finish`` (``lngram_v2.py:1354-1359``): ``mixed = W_o head``; ``mixed + conv(mixed)``."""
    b, t = head.shape[:2]
    mixed = F.linear(head.reshape(b, t, -1), _p(params, "readout_o_proj.weight", head.dtype))
    return mixed + causal_conv(params, cfg, mixed, segment_ids)


def memory_forward(params: dict, cfg: MemCfg, h: torch.Tensor, codes, segment_ids=None,
                   dtype: torch.dtype | None = None) -> torch.Tensor:
    """``RouteNgramMemoryV2.forward`` in ``full`` mode, eval (``lngram_v2.py:1361-1407``):
    query from ``h``, route tokens from ``codes``, project, sink GQA, finish."""
    dt = dtype or h.dtype
    h = h.to(dt)
    tables = {n: params[f"tables.ngram_{n}.weight"].to(dt) for n in cfg.orders}
    q = project_query(params, cfg, h)
    tok = route_tokens(tables, codes, cfg.orders, cfg.bits, segment_ids=segment_ids)
    key, value = project_memory(params, cfg, tok)
    head = manual_gqa(cfg, q, key, value)
    return finish(params, cfg, head, segment_ids)


def router_logits(x: torch.Tensor, w: torch.Tensor, work=torch.float64) -> torch.Tensor:
    """``LngramMemory.route_logits`` (``wrapper.py:98-101``): ``F.linear(x.float(), W.float())``.

    ``work=float64`` gives the exact-product, near-exact-sum oracle (for bf16 operands
    every product is exact); ``work=float32`` is the reference's own precision.
    """
    return F.linear(x.to(work), w.to(work))


def lngram_forward(params: dict, cfg: MemCfg, h: torch.Tensor, h_norm: torch.Tensor,
                   router_in: torch.Tensor | None = None, dtype: torch.dtype | None = None,
                   codes=None):
    """``LngramMemory.forward`` in eval (``wrapper.py:103-125``): router logits on
    ``h_norm`` (or ``router_in``), sign-packed codes, module forward with the raw ``h``.

    ``codes`` (optional) replaces the router's codes, so outputs can be compared given
    identical codes.  Returns ``(out, codes, q_logits_fp64)``.
    """
    x = h_norm if router_in is None else router_in
    q = router_logits(x, params["router.weight"].to(x.dtype))
    if codes is None:
        codes = pack_route_codes(q.numpy(), cfg.bits)
    out = memory_forward(params, cfg, h, codes, dtype=dtype)
    return out, codes, q


# ----------------------------------------------------------------------------- SD router / SSM
def router_features(emb: torch.Tensor, start: torch.Tensor, prev_w: torch.Tensor, cur_w: torch.Tensor,
                    eps: float, ssm_state: torch.Tensor | None = None) -> torch.Tensor:
    """``TokenRouterFeatures.forward`` (``router.py:50-59``): ``concat(RMSNorm(E[x_{t-1}]
    or start), RMSNorm(E[x_t])[, s_t cast to the feature dtype])``."""
    b = emb.shape[0]
    prev = torch.cat((start.to(emb.dtype).expand(b, 1, -1), emb[:, :-1]), 1)
    parts = [rms_norm(prev, prev_w, eps), rms_norm(emb, cur_w, eps)]
    if ssm_state is not None:
        parts.append(ssm_state.to(parts[0].dtype))
    return torch.cat(parts, -1)


def ssm_inputs(emb: torch.Tensor, norm_w: torch.Tensor, w_in: torch.Tensor, eps: float,
               work=torch.float32) -> torch.Tensor:
    """``DiagonalSSM.inputs`` (``ssm.py:41-43``): ``W_in RMSNorm(E[x])`` in fp32."""
    x = emb.to(work)
    xn = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return F.linear(xn * norm_w.to(work), w_in.to(work))


def ssm_scan(a, u, s0=None) -> np.ndarray:
    """Diagonal SSM states (``ssm.py:58-65`` sequential form, ``infer.py:125-137`` for a
    carried state): ``s_t = a s_{t-1} + (1-a) u_t``, ``s_{-1} = s0`` (zero if None), in fp64.

    a ``[N]``, u ``[B, T, N]``, s0 ``[B, N]`` -> s ``[B, T, N]`` (numpy fp64).
    """
    a = np.asarray(a, np.float64)
    u = np.asarray(u, np.float64)
    b, t, n = u.shape
    s = np.zeros((b, n)) if s0 is None else np.asarray(s0, np.float64).copy()
    out = np.empty((b, t, n))
    for i in range(t):
        s = a * s + (1.0 - a) * u[:, i]
        out[:, i] = s
    return out


def ssm_scan_closed_form_constant(a, u_const, t: int, s0=None) -> np.ndarray:
    """Closed form of the recurrence for a constant input: ``s_t = u + a^{t+1} (s0 - u)``."""
    a = np.asarray(a, np.float64)
    u = np.asarray(u_const, np.float64)
    s0 = np.zeros_like(u) if s0 is None else np.asarray(s0, np.float64)
    k = np.arange(1, t + 1, dtype=np.float64)[:, None]
    return u[None] + (a[None] ** k) * (s0 - u)[None]


# ----------------------------------------------------------------------------- draft-tree verification
def tree_paths(parent) -> list:
    """Root-to-node paths of a tree given by ``parent`` (``parent[0] = -1``, ``parent[i] < i``;
    ``drafting/tree.py:37-51``)."""
    paths = []
    for i, p in enumerate(parent):
        if p < 0:
            paths.append([i])
        else:
            if not 0 <= p < i:
                raise ValueError("parent[i] must lie in [0, i)")
            paths.append(paths[p] + [i])
    return paths


def ssm_tree(a, u, parent, s_root=None) -> np.ndarray:
    """SSM states of the tree nodes in ``tree_verify_step`` (``drafting/tree.py:153-161``):
    ``s_i = a s_parent(i) + (1-a) u_i``, the root continuing from ``s_root`` (the cached state at
    ``L - 1``, zero if None), in fp64.  a ``[N]``, u ``[B, n, N]`` -> ``[B, n, N]``."""
    a = np.asarray(a, np.float64)
    u = np.asarray(u, np.float64)
    b, n, c = u.shape
    root = np.zeros((b, c)) if s_root is None else np.asarray(s_root, np.float64)
    out = np.empty((b, n, c))
    for i, p in enumerate(parent):
        sp = root if p < 0 else out[:, p]
        out[:, i] = a * sp + (1.0 - a) * u[:, i]
    return out


def tree_memory_forward(params: dict, cfg: MemCfg, h_hist: torch.Tensor, codes_hist, h_nodes: torch.Tensor,
                        codes_nodes, parent, dtype: torch.dtype | None = None) -> torch.Tensor:
    """The memory block of ``tree_verify_step`` (``drafting/tree.py:179-196``) for tree nodes after
    ``L`` cached positions: node i's n-gram windows (``tree_ngram_codes`` :114-127) and conv window
    (``tree_slots`` :96-111, :186-194) follow its ancestors and then the cached history, so its
    output is the sequence forward's at the last position of history + its root path.  h_hist
    ``[B, L, d]`` with codes ``[B, L, R]``; h_nodes ``[B, n, d]`` with codes ``[B, n, R]`` ->
    ``[B, n, d]``."""
    ch = np.asarray(codes_hist)
    cn = np.asarray(codes_nodes)
    outs = []
    for path in tree_paths(parent):
        hs = torch.cat((h_hist, h_nodes[:, path]), 1)
        cs = np.concatenate((ch, cn[:, path]), 1)
        outs.append(memory_forward(params, cfg, hs, cs, dtype=dtype)[:, -1])
    return torch.stack(outs, 1)


# ----------------------------------------------------------------------------- lookup surrogate (training)
def surrogate_grad(grad_memory: torch.Tensor, hard_memory: torch.Tensor, q_logits: torch.Tensor, codes, table,
                   valid, order: int, bits: int, route_start: int, temperature: float, scale: float, exact: bool,
                   work=torch.float64) -> torch.Tensor:
    """Route-logit gradient of ``_LngramSurrogate.backward`` (``lngram_v2.py:364-464``) for one order.

    Window ``w = 0 .. T-order`` ends at position ``w + order - 1`` and reads row ``idx_w``
    (``route_rows``); its masked memory gradient is ``g_w`` and its looked-up row ``m_w``.
    Digit ``e`` of the window is the code at position ``w + e``, so that position collects:

    - approximate (``:430-447``): per bit k, ``sign * (table[idx_w ^ 2^(e*bits+k)] . g_w - m_w . g_w)``
      (sign +1 when the bit is 0), the total scaled by ``scale * T * p (1-p)``;
    - exact (``:394-429``): ``scale * T * sum_code P(code) (bit_k(code) - p_k) (table[row_w(e <- code)] . g_w)``
      with ``P`` the product of the position's bit probabilities, ``p = sigmoid(T q)``.

    ``valid`` is ``_valid_mask`` ``[B, T]``.  Returns ``[B, T, R, bits]`` in ``work``.
    """
    b, t, r, nb = q_logits.shape
    A = 1 << bits
    n_win = t - order + 1
    out = torch.zeros(b, t, r, nb, dtype=work)
    if n_win <= 0 or temperature == 0.0 or scale == 0.0:
        return out
    c = np.asarray(codes).astype(np.int64)
    base = np.arange(route_start, route_start + r, dtype=np.int64)[None, None, :] * A ** order
    idx = base + ngram_address(c, order, bits)                                  # [B, n_win, R]
    keep = torch.as_tensor(np.asarray(valid, bool)[:, order - 1:]).to(work)
    g = grad_memory[:, order - 1:].to(work) * keep[..., None, None]
    tab = table.to(work)
    p = torch.sigmoid(temperature * q_logits.to(work))
    ts = scale * temperature

    def dots(rows: np.ndarray) -> torch.Tensor:
        return (tab[torch.from_numpy(rows)] * g).sum(-1)                       # [B, n_win, R]

    for e in range(order):
        at = slice(e, e + n_win)                                               # positions w + e
        if exact:
            digit = c[:, e:e + n_win] & (A - 1)
            pe = p[:, at]
            for code in range(A):
                d = dots(idx + (code - digit) * A ** e)
                bit = torch.tensor([(code >> k) & 1 for k in range(nb)], dtype=work)
                prob = torch.where(bit.bool(), pe, 1.0 - pe).prod(-1)
                out[:, at] += ts * prob[..., None] * (bit - pe) * d[..., None]
        else:
            here = (hard_memory[:, order - 1:].to(work) * g).sum(-1)
            for k in range(nb):
                flip = 1 << (e * bits + k)
                sign = torch.from_numpy(1.0 - 2.0 * ((idx & flip) != 0)).to(work)
                out[:, at, :, k] += (dots(idx ^ flip) - here) * sign
    if not exact:
        out *= ts * p * (1.0 - p)
    return out


def surrogate_expected_dot(q_logits: torch.Tensor, codes, table, grad_memory: torch.Tensor, valid, order: int,
                           bits: int, route_start: int, temperature: float, scale: float) -> torch.Tensor:
    """The objective whose exact derivative the exact surrogate mode is, computed by brute force
    in fp64 (a check, not a restatement): ``scale * sum over windows w, digits e and codes c of
    P(c | sigmoid(T q[w+e])) * (table[row of w with digit e replaced by c] . g_w)``, the other
    digits held at their codes.  Differentiating it in ``q`` gives ``_LngramSurrogate``'s exact mode
    (``lngram_v2.py:394-429``)."""
    b, t, r, nb = q_logits.shape
    A = 1 << bits
    c = np.asarray(codes).astype(np.int64)
    tab = table.double()
    p = torch.sigmoid(temperature * q_logits.double())
    total = torch.zeros((), dtype=torch.float64)
    vm = np.asarray(valid, bool)
    for bi in range(b):
        for w in range(t - order + 1):
            end = w + order - 1
            if not vm[bi, end]:
                continue
            for ri in range(r):
                g = grad_memory[bi, end, ri].double()
                digits = [int(c[bi, w + k, ri]) for k in range(order)]
                for e in range(order):
                    pe = p[bi, w + e, ri]
                    for code in range(A):
                        dg = list(digits)
                        dg[e] = code
                        row = (route_start + ri) * A ** order + sum(v << (k * bits) for k, v in enumerate(dg))
                        prob = torch.ones((), dtype=torch.float64)
                        for k in range(nb):
                            prob = prob * (pe[k] if (code >> k) & 1 else 1.0 - pe[k])
                        total = total + prob * (tab[row] @ g)
    return scale * total


# ----------------------------------------------------------------------------- comparison metric
def rel_err(got, want) -> float:
    """Norm-relative error ``||got - want|| / ||want||`` in fp64."""
    g = torch.as_tensor(got).double()
    w = torch.as_tensor(want).double()
    den = float(w.norm())
    return float((g - w).norm()) / (den if den > 0 else 1.0)
