"""Draft readout from the memory table alone: drop-in for the reference ``ffnmem/memory/draft.py``.

Per drafted position t: route tokens of the n-grams ending at t, the shared memory
norm + KV projection, a query ``W_q RMSNorm(E[x_t]) (+ W_sq s_t)``, sink attention
over the R routes, ``W_o`` -> RMSNorm, and logits against the tied embedding
(``draft.py:1-91``).  Every op is a gfx950 kernel.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from lngram_hip import ops

from ..model import RMSNorm
from .lngram_v2 import RouteNgramMemoryV2


def lookup_rows_at(m: RouteNgramMemoryV2, codes: Tensor, q_logits: Tensor | None, b_idx: Tensor,
                   t_idx: Tensor) -> Tensor:
    """Route tokens ``[N, R, len(ngrams)*mem_dim]`` of the n-grams ending at ``(b_idx[i], t_idx[i])``
    (``draft.py:26-47``), equal to the full lookup at those positions.  The codes are padded with
    ``route_history_length`` slots before position 0; each position's window is the slice of the
    padded sequence that ends at it, and the pad slots are not real, so an n-gram that reaches
    before the sequence start reads the zero row.  ``q_logits`` (the training surrogate's input) is
    not used in eval."""
    from drafting.drafters import window_route_tokens

    hist = m.route_history_length
    padded = F.pad(codes, (0, 0, hist, 0))                     # slot hist + t holds position t
    span = t_idx[:, None] + torch.arange(hist + 1, device=codes.device)[None, :]
    return window_route_tokens(m, padded[b_idx[:, None], span], span >= hist)


class DraftReadout(nn.Module):
    """``DraftReadout`` (``draft.py:50-91``); parameters ``q_norm``, ``w_q``, ``w_sq``, ``w_o``, ``out_norm``."""

    def __init__(self, d_model: int, memory_module: RouteNgramMemoryV2, q_heads: int = 4, head_dim: int = 64,
                 ssm_dim: int = 0, eps: float = 1e-5, init_std: float = 0.02):
        super().__init__()
        kv_heads = memory_module.readout_num_kv_heads
        if head_dim != memory_module.readout_head_dim:
            raise ValueError(f"draft head_dim {head_dim} != memory readout head_dim {memory_module.readout_head_dim}")
        if q_heads % kv_heads:
            raise ValueError(f"draft q_heads {q_heads} not a multiple of memory kv_heads {kv_heads}")
        self.q_heads, self.head_dim, self.kv_heads = q_heads, head_dim, kv_heads
        self.groups = q_heads // kv_heads
        inner = q_heads * head_dim
        self.q_norm = RMSNorm(d_model, eps)
        self.w_q = nn.Linear(d_model, inner, bias=False)
        self.w_sq = nn.Linear(ssm_dim, inner, bias=False) if ssm_dim else None
        self.w_o = nn.Linear(inner, d_model, bias=False)
        self.out_norm = RMSNorm(d_model, eps)
        for lin in (self.w_q, self.w_sq, self.w_o):
            if lin is not None:
                nn.init.normal_(lin.weight, mean=0.0, std=init_std)

    def hidden(self, m: RouteNgramMemoryV2, emb_cur: Tensor, route_tokens: Tensor,
               ssm_state: Tensor | None = None) -> Tensor:
        """``emb_cur [N, d]``, ``route_tokens [N, R, D]`` -> draft hidden ``[N, d]``."""
        n = emb_cur.shape[0]
        q = ops.linear(self.q_norm(emb_cur), self.w_q.weight)
        if self.w_sq is not None:
            q = q + ops.linear(ssm_state.to(q.dtype), self.w_sq.weight)
        key, value = m._project_memory(route_tokens[:, None])  # [N, 1, kv, R, hd]
        grouped = q.view(n, 1, self.kv_heads, self.groups, self.head_dim).to(key.dtype)
        out = ops.sink_attention(grouped, key, value, m.softmax_scale, m.readout_sink_logit)
        out = out.reshape(n, self.q_heads * self.head_dim)
        return self.out_norm(ops.linear(out, self.w_o.weight))

    def forward(self, m: RouteNgramMemoryV2, emb_cur: Tensor, route_tokens: Tensor, unembed: Tensor,
                ssm_state: Tensor | None = None) -> Tensor:
        """Draft logits ``[N, V]``; ``unembed`` is the tied embedding ``[V, d]``."""
        h = self.hidden(m, emb_cur, route_tokens, ssm_state)
        return ops.linear(h, unembed.to(h.dtype))
