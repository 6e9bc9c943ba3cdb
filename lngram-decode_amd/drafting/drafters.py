"""Window helpers and code-keyed online counts of the reference's ``drafting/drafters.py``
(``window_rows :99-107``, ``window_route_tokens :110-114``, ``OnlineCounts :117-142``), on the GPU.

A window is the last ``W`` route codes before a drafted position, ``win [N, W, R]``, with
``real [N, W]`` marking the slots that hold a position of the sequence.  Slots that are not real
always form a prefix of the window (positions before the sequence start), so an n-gram ending at
the window's last slot is valid exactly when its first slot is real.

The offline acceptance harness built on these (``WindowDrafter`` and its subclasses, which drive a
backbone target over evaluation records) is evaluation tooling, not part of this path.
"""

from __future__ import annotations

import torch
from torch import Tensor

from lngram_hip import ops


def _window_masks(win: Tensor, real: Tensor) -> tuple[Tensor, Tensor]:
    """(segment ids, valid tokens) under which the v2 validity rule reads a prefix-masked window:
    a row is valid iff its first and last slots share a segment and its last slot is a token."""
    seg = real.to(torch.int32)
    return seg, real.to(torch.uint8)


def window_rows(win: Tensor, real: Tensor, order: int, bits: int) -> Tensor:
    """Global rows ``[N, R]`` (int64) of the order-``order`` n-gram ending at each window's last slot,
    -1 where it reaches a slot that is not real."""
    seg, val = _window_masks(win, real)
    rows = ops.ngram_rows(win * real[..., None].to(win.dtype), [int(order)], bits, segment_ids=seg,
                          valid_tokens=val, rows_dtype=torch.int64)
    return rows[:, -1, :, 0]


def window_route_tokens(m, win: Tensor, real: Tensor) -> Tensor:
    """Memory route tokens ``[N, R, Dt]`` of the n-grams ending at each window's last slot (zero rows
    for n-grams that reach a slot that is not real).  ``m`` is the ``RouteNgramMemoryV2``."""
    seg, val = _window_masks(win, real)
    tables = [m.tables[f"ngram_{n}"].weight for n in m.ngrams]
    tok = ops.route_tokens(win * real[..., None].to(win.dtype), tables, m.ngrams, m.bits_per_route, 0,
                           m.num_routes, seg, val, 1)
    return tok[:, -1]


class OnlineCounts:
    """In-context (order, route, row) -> next-token counts of one sequence's committed pairs
    (``drafters.py:117-142``): keys are the rows of the n-grams ending at t, paired with token t + 1,
    for t = 0 .. T-2.  ``mix`` runs ``lng_online_mix``."""

    def __init__(self, codes: Tensor, x: Tensor, orders, bits: int, vocab: int, kappa: float = 1.0,
                 route_chunk: int = 32):
        if codes.dim() != 2 or x.dim() != 1 or codes.shape[0] != x.shape[0]:
            raise ValueError("OnlineCounts: codes [T, R] and tokens [T]")
        self.orders, self.bits, self.vocab, self.kappa = tuple(int(n) for n in orders), int(bits), int(vocab), kappa
        self.rc = route_chunk  # the reference's memory chunking; the kernel needs none
        self.routes = codes.shape[1]
        self.keys = ops.ngram_rows(codes[None], self.orders, self.bits, rows_dtype=torch.int32)[0, :-1]
        self.nxt = x[1:].to(torch.int64)

    def mix(self, p: Tensor, win: Tensor, real: Tensor, deadline: Tensor) -> Tensor:
        """``p [N, V]`` mixed with the counts of the pairs ``t <= deadline[j]`` matching row j's window."""
        q = torch.stack([window_rows(win, real, n, self.bits) for n in self.orders], -1).to(torch.int32)
        return ops.online_mix(self.keys, self.nxt, q, deadline, p, self.kappa)
