"""Drafter API entry points (``drafting/cpu_drafter.py`` of the reference): ``DraftOut`` and
``make_drafter``.  On this path every drafter runs on the GPU (``GpuDrafter``), whichever
implementation a caller asks for; the reference's CPU implementations (``RefDrafter`` in PyTorch,
``CppDrafter`` in C++) are not part of it."""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass
class DraftOut:
    """``DraftOut`` (``cpu_drafter.py:51-61``)."""

    tokens: list            # gamma drafted tokens (top-1 chain)
    topk_ids: np.ndarray    # int64 [gamma, k] (-1 = fewer candidates)
    topk_logits: np.ndarray  # float32 [gamma, k] (-inf pad)
    codes: np.ndarray       # uint8 [len(hyp) + advanced drafts, R]

    @property
    def runner_up(self) -> int:
        """Runner-up at the first drafted position (repair branch), -1 if none."""
        return int(self.topk_ids[0, 1]) if self.topk_ids.shape[1] > 1 else -1


def make_drafter(bundle, impl: str = "auto", **kw):
    """``make_drafter`` (``cpu_drafter.py:392-397``).  Every ``impl`` the reference accepts -- ``ref``
    (its PyTorch drafter), ``cpp`` (its C++ drafter), ``auto`` -- and ``gpu`` build the GPU drafter,
    which has the same API and results; ``threads`` (the C++ drafter's worker count) has no
    meaning on the GPU and is dropped."""
    if impl not in ("ref", "cpp", "auto", "gpu"):
        raise ValueError(f"impl must be ref | cpp | auto | gpu, got {impl!r}")
    kw.pop("threads", None)
    from .gpu_drafter import GpuDrafter

    return GpuDrafter(bundle, **kw)
