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
        self._tables_cache = None

    def _features(self, emb: Tensor, ssm_state: Tensor | None, token_ids: Tensor | None = None) -> Tensor:
        if self.kind == "embed2_ssm" and ssm_state is None:
            raise ValueError("embed2_ssm router needs the SSM state")
        s = ssm_state if self.kind == "embed2_ssm" else None
        n = 0 if s is None else s.shape[-1]
        if not ops.router_features_ok(emb.shape[-1], n, emb.dtype):
            raise NotImplementedError(f"lng_router_features takes fp32/bf16 features whose rows are 16-byte "
                                      f"multiples up to 8 KB (d={emb.shape[-1]}, state {n}, {emb.dtype})")
        return ops.router_features(emb, self.start, self.prev_norm.weight, self.cur_norm.weight, self.prev_norm.eps,
                                   ssm_state=s, token_ids=token_ids)

    def forward(self, emb: Tensor, ssm_state: Tensor | None = None) -> Tensor:
        """emb ``[B, T, d]``; ssm_state ``[B, T, N]`` for ``embed2_ssm`` -> ``[B, T, 2d (+ N)]``, one
        ``lng_router_features`` launch."""
        return self._features(emb, ssm_state)

    def from_ids(self, token_ids: Tensor, table: Tensor, ssm_state: Tensor | None = None) -> Tensor:
        """``forward(table[token_ids], ssm_state)`` with the embedding gather fused into the kernel
        (not in the reference module: the model gathers ``emb`` itself)."""
        return self._features(table, ssm_state, token_ids)

    def tables(self, table: Tensor) -> tuple:
        """``(fprev, fcur)``: the normalised rows of the embedding table for the previous-token and the
        current-token halves (``fprev[V]`` the normalised ``start``, a zero row last in each;
        ``ops.router_feature_tables``), cached per version of the table and of this module's
        parameters.  Not in the reference module: the gathered router GEMM reads them."""
        ps = (table, self.start, self.prev_norm.weight, self.cur_norm.weight)
        key = tuple((p.data_ptr(), p._version) for p in ps) + (table.shape, table.device)
        if self._tables_cache is None or self._tables_cache[0] != key:
            with torch.no_grad():
                t = ops.router_feature_tables(table.detach(), self.start.detach(), self.prev_norm.weight.detach(),
                                              self.cur_norm.weight.detach(), self.prev_norm.eps)
            self._tables_cache = (key, t)
        return self._tables_cache[1]

    def step(self, emb_prev: Tensor | None, emb_cur: Tensor, ssm_state: Tensor | None = None) -> Tensor:
        """Single positions (decode / drafter / tree nodes): ``[..., d]`` inputs, every leading index an
        independent (previous, current) pair, as the reference's elementwise ``step``
        (``router.py:61-68``); ``emb_prev`` None at t = 0.  The kernel runs on each two-position
        sequence (previous, current) and the last position is kept: its previous-token half reads
        ``emb_prev`` (at t = 0 the one-position sequence reads ``start``)."""
        lead, d = emb_cur.shape[:-1], emb_cur.shape[-1]
        cur = emb_cur.reshape(-1, d)
        seq = cur[:, None] if emb_prev is None else torch.stack((emb_prev.reshape(-1, d).to(cur.dtype), cur), 1)
        s = None
        if self.kind == "embed2_ssm":
            if ssm_state is None:
                raise ValueError("embed2_ssm router needs the SSM state")
            s = ssm_state.reshape(cur.shape[0], -1)[:, None].expand(-1, seq.shape[1], -1)
        out = self._features(seq, s)[:, -1]
        return out.reshape(*lead, out.shape[-1])


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
