"""The backbone's ``RMSNorm`` (``ffnmem/model.py:39-48``), the one norm of that module on this
path: the memory's token router features (``router.py:40``), the SSM input (``ssm.py:27``) and
the draft head (``draft.py:54``) import it from here, as in the reference.  The rest of the
backbone is not part of the MI355X build.

It rounds differently from the memory module's own ``lngram_v2.RMSNorm``: the normalised row is
rounded to the input dtype before the weight multiplies it, and the product is rounded again.
"""

from __future__ import annotations

import torch
from torch import Tensor, nn

from lngram_hip import ops


class RMSNorm(nn.Module):
    """``RMSNorm(dim, eps)``; parameter ``weight`` (ones).  Runs ``lng_rmsnorm`` (``LNG_NORM_MODEL``)."""

    def __init__(self, dim: int, eps: float):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: Tensor) -> Tensor:
        if x.shape[-1] != self.weight.shape[0]:
            raise ValueError(f"RMSNorm expects last dim {self.weight.shape[0]}, got {x.shape[-1]}")
        return ops.rmsnorm(x, self.weight, self.eps)
