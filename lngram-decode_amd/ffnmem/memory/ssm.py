"""Non-selective diagonal SSM over token embeddings (SD-C): drop-in for ``ffnmem/memory/ssm.py``.

    u[t] = W_in RMSNorm(E[x[t]])          (fp32)
    a    = sigmoid(theta)
    s[t] = a * s[t-1] + (1 - a) * u[t],    s[-1] = 0

Both scan functions of the reference (``chunked_scan`` and ``sequential_scan``,
``ssm.py:58-91``) compute the same recurrence; here both run ``lng_ssm_scan`` (one pass
over the inputs, tiles of 128 steps chained by a decoupled look-back on the GPU).
"""

from __future__ import annotations

import math

import torch
from torch import Tensor, nn

from lngram_hip import ops

from ..model import RMSNorm


class DiagonalSSM(nn.Module):
    """``ssm.py:22-55``; parameters ``norm.weight``, ``w_in.weight``, ``theta``."""

    def __init__(self, d_model: int, state_dim: int = 256, chunk: int = 128, eps: float = 1e-5,
                 init_std: float = 0.02, decay_min: float = 0.5, decay_max: float = 0.999):
        super().__init__()
        self.state_dim, self.chunk = int(state_dim), int(chunk)
        self.norm = RMSNorm(d_model, eps)
        self.w_in = nn.Linear(d_model, self.state_dim, bias=False)
        nn.init.normal_(self.w_in.weight, mean=0.0, std=init_std)
        # geometric spacing of the time constants 1/(1-a) between the two decays
        one_minus = torch.exp(torch.linspace(math.log(1 - decay_min), math.log(1 - decay_max), self.state_dim))
        a = 1.0 - one_minus
        self.theta = nn.Parameter(torch.log(a) - torch.log1p(-a))

    def decay(self) -> Tensor:
        return torch.sigmoid(self.theta.float())

    def inputs(self, emb: Tensor) -> Tensor:
        """``u[t]`` in fp32: ``[B, T, d]`` -> ``[B, T, N]`` (``ssm.py:41-43``)."""
        x = emb.float()
        return ops.linear(ops.rmsnorm(x, self.norm.weight.float(), self.norm.eps), self.w_in.weight.float())

    def forward(self, emb: Tensor) -> Tensor:
        return chunked_scan(self.decay(), self.inputs(emb), self.chunk)

    def step(self, state: Tensor | None, emb_t: Tensor) -> Tensor:
        """One recurrence step: ``emb_t [B, d]``, ``state [B, N]`` or None -> new state."""
        u = self.inputs(emb_t[:, None])
        return ops.ssm_scan(self.decay(), u, state)[:, 0]


def sequential_scan(a: Tensor, u: Tensor) -> Tensor:
    """``a [N]``, ``u [B, T, N]`` -> ``s [B, T, N]`` (``ssm.py:58-65``)."""
    return ops.ssm_scan(a, u)


def chunked_scan(a: Tensor, u: Tensor, chunk: int = 128) -> Tensor:
    """Same result as ``sequential_scan`` (``ssm.py:68-91``); ``chunk`` is accepted for API
    compatibility (the kernel picks its own chunking)."""
    if int(chunk) <= 0:
        raise ValueError("chunk must be positive")
    return ops.ssm_scan(a, u)


def scan_from(a: Tensor, u: Tensor, s_prev: Tensor | None) -> Tensor:
    """States for new positions given the state before them (``infer.py:125-137`` ``ssm_continue``)."""
    return ops.ssm_scan(a, u, s_prev)
