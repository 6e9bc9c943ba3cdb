"""Token-only router inputs (SD-B / SD-C): drop-in for the reference ``ffnmem/memory/router.py``.

``router_input``: ``hidden`` (router reads the block's pre-attention RMSNorm output),
``embed2`` = ``concat(RMSNorm(E[x[t-1]]), RMSNorm(E[x[t]]))`` or ``embed2_ssm`` which
appends the SSM state ``s[t]`` (``router.py:1-34``).  A learned ``start`` vector
stands in for ``E[x[-1]]``.
"""

from __future__ import annotations

import torch
from torch import Tensor, nn

from lngram_hip import ops

from ..model import RMSNorm

ROUTER_INPUTS = ("hidden", "embed2", "embed2_ssm")


def router_input_dim(kind: str, d_model: int, ssm_dim: int) -> int:
    """``router.py:25-34``."""
    if kind == "hidden":
        return d_model
    if kind == "embed2":
        return 2 * d_model
    if kind == "embed2_ssm":
        if ssm_dim <= 0:
            raise ValueError("router_input embed2_ssm needs model.ssm")
        return 2 * d_model + ssm_dim
    raise ValueError(f"router_input must be one of {ROUTER_INPUTS}, got {kind!r}")


class TokenRouterFeatures(nn.Module):
    """``router.py:37-68``; parameters ``prev_norm.weight``, ``cur_norm.weight``, ``start``."""

    def __init__(self, d_model: int, kind: str, eps: float = 1e-5, init_std: float = 0.02):
        super().__init__()
        if kind not in ("embed2", "embed2_ssm"):
            raise ValueError(f"TokenRouterFeatures does not handle {kind!r}")
        self.kind = kind
        self.prev_norm = RMSNorm(d_model, eps)
        self.cur_norm = RMSNorm(d_model, eps)
        self.start = nn.Parameter(torch.empty(d_model))
        nn.init.normal_(self.start, mean=0.0, std=init_std)

    def forward(self, emb: Tensor, ssm_state: Tensor | None = None) -> Tensor:
        """emb ``[B, T, d]``; ssm_state ``[B, T, N]`` for ``embed2_ssm``."""
        if self.kind == "embed2_ssm" and ssm_state is None:
            raise ValueError("embed2_ssm router needs the SSM state")
        s = ssm_state if self.kind == "embed2_ssm" else None
        n = 0 if s is None else s.shape[-1]
        if ops.router_features_ok(emb.shape[-1], n, emb.dtype):
            return ops.router_features(emb, self.start, self.prev_norm.weight, self.cur_norm.weight, self.prev_norm.eps,
                                       ssm_state=s)
        b = emb.shape[0]
        prev = torch.cat((self.start.to(emb.dtype).expand(b, 1, -1), emb[:, :-1]), dim=1)
        parts = [self.prev_norm(prev), self.cur_norm(emb)]
        if s is not None:
            parts.append(s.to(parts[0].dtype))
        return torch.cat(parts, dim=-1)

    def from_ids(self, token_ids: Tensor, table: Tensor, ssm_state: Tensor | None = None) -> Tensor:
        """``forward(table[token_ids], ssm_state)`` with the embedding gather fused into the kernel
        (not in the reference module: the model gathers ``emb`` itself)."""
        if self.kind == "embed2_ssm" and ssm_state is None:
            raise ValueError("embed2_ssm router needs the SSM state")
        return ops.router_features(table, self.start, self.prev_norm.weight, self.cur_norm.weight, self.prev_norm.eps,
                                   ssm_state=ssm_state if self.kind == "embed2_ssm" else None, token_ids=token_ids)

    def step(self, emb_prev: Tensor | None, emb_cur: Tensor, ssm_state: Tensor | None = None) -> Tensor:
        """One position (decode / drafter): ``emb_prev`` None at t = 0."""
        if emb_prev is None:
            emb_prev = self.start.to(emb_cur.dtype).expand_as(emb_cur)
        parts = [self.prev_norm(emb_prev), self.cur_norm(emb_cur)]
        if self.kind == "embed2_ssm":
            parts.append(ssm_state.to(parts[0].dtype))
        return torch.cat(parts, dim=-1)


class TokenRouter(nn.Module):
    """SD-A imitating router (``router.py:71-84``): embed2 features -> ``R*bits`` fp32 logits."""

    def __init__(self, d_model: int, out_dim: int, eps: float = 1e-5, init_std: float = 0.02):
        super().__init__()
        self.features = TokenRouterFeatures(d_model, "embed2", eps, init_std)
        self.proj = nn.Linear(2 * d_model, out_dim, bias=False)
        nn.init.normal_(self.proj.weight, mean=0.0, std=init_std)

    def forward(self, emb: Tensor) -> Tensor:
        x = self.features(emb)
        logits, _ = ops.router_codes(x, self.proj.weight, 1, want_logits=True)
        return logits
