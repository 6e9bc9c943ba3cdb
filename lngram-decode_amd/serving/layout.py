"""Serving row layout of the n-gram tables: drop-in for the reference ``serving/layout.py``
(``reverse_digits`` :26-35, ``permute_table`` :38-43, ``permute_tables`` :46-49, ``serving_address``
:52-63, ``serving_route_tokens`` :66-81, ``candidate_base`` :84-100, ``candidate_rows`` :103-108,
``select_candidates`` :111-116).

The v2 tables address an n-gram with its oldest code least significant, so the 2^bits rows that
the next step may read lie 2^bits or 2^(2 bits) rows apart.  The serving layout reverses the n
base-2^bits digits of every in-route index (an involution), putting the current code least
significant: the candidates of the next step are one contiguous block of 2^bits rows.  Only the
row order changes; the route tokens equal the v2 lookup's.

The movers are gfx950 kernels (``lng_permute_table``, ``lng_serving_address``,
``lng_serving_gather``, ``lng_serving_candidates``, ``lng_select_candidates``); the tables they
read may sit in device memory or in pinned host memory, which the kernels read directly.
``reverse_digits`` and ``candidate_base`` are index bookkeeping on any device.
"""

from __future__ import annotations

import torch
from torch import Tensor

from lngram_hip import ops


def reverse_digits(n_digits: int, bits: int, device=None) -> Tensor:
    """Index map ``j -> j`` with its ``n_digits`` base-2^bits digits in reverse order (an involution)."""
    a = 1 << bits
    j = torch.arange(a ** n_digits, device=device, dtype=torch.long)
    out = torch.zeros_like(j)
    for k in range(n_digits):
        out += ((j >> (k * bits)) & (a - 1)) << ((n_digits - 1 - k) * bits)
    return out


def permute_table(weight: Tensor, routes: int, order: int, bits: int) -> Tensor:
    """v2 table ``[R * 16^n, D]`` -> serving layout (same shape); also the way back."""
    return ops.permute_table(weight, int(routes), int(order), int(bits))


def permute_tables(module) -> dict[int, Tensor]:
    """Serving-layout copies of every order's table of a ``RouteNgramMemoryV2``."""
    return {order: permute_table(module.tables[f"ngram_{order}"].weight.detach(), module.num_routes, order,
                                 module.bits_per_route)
            for order in module.ngrams}


def serving_address(codes: Tensor, order: int, bits: int) -> Tensor:
    """Addresses ``[B, T-order+1, R]`` of the n-grams ending at ``t = order-1 .. T-1``, current code
    least significant."""
    return ops.serving_address(codes, int(order), int(bits))


def serving_route_tokens(tables: dict, codes: Tensor, ngrams, bits: int) -> Tensor:
    """Route tokens ``[B, T, R, len(ngrams) * D]`` from serving-layout tables (zeros where the n-gram
    does not fit), equal to v2's ``_lookup_route_chunk`` without masking."""
    orders = [int(o) for o in ngrams]
    return ops.serving_gather([tables[o] for o in orders], orders, int(bits), codes, codes.shape[1], 0)


def candidate_base(history: Tensor, order: int, bits: int) -> Tensor:
    """First row ``[B, R]`` of the 2^bits candidates of the next step, per route: ``history [B, order-1,
    R]`` holds the codes ending at the current step, oldest first; the candidates are rows
    ``base .. base + 2^bits - 1``, indexed by the next code."""
    b, h, r = history.shape
    if h != order - 1:
        raise ValueError(f"need {order - 1} history codes for order {order}, got {h}")
    suffix = torch.zeros(b, r, dtype=torch.long, device=history.device)
    for m in range(1, order):                      # code t - m + 1 is digit m
        suffix += (history[:, h - m].to(torch.long) & ((1 << bits) - 1)) << (m * bits)
    return torch.arange(r, device=history.device).view(1, r) * (1 << (bits * order)) + suffix


def candidate_rows(tables: dict, history: Tensor, ngrams, bits: int) -> dict[int, Tensor]:
    """Contiguous candidate blocks of the next step: ``{order: [B, R, 2^bits, D]}`` from ``history [B, H,
    R]`` (the last max(ngrams) - 1 codes, oldest first)."""
    orders = [int(o) for o in ngrams]
    h = history.shape[1]
    if h < max(orders) - 1:
        raise ValueError(f"need {max(orders) - 1} history codes, got {h}")
    cand = ops.serving_candidates([tables[o] for o in orders], orders, int(bits), history, h)
    return {o: cand[:, :, k] for k, o in enumerate(orders)}


def select_candidates(cands: dict, next_codes: Tensor, ngrams) -> Tensor:
    """Rows ``[B, R, len(ngrams) * D]`` of the actual next codes ``[B, R]`` from candidate blocks."""
    orders = [int(o) for o in ngrams]
    blocks = torch.stack([cands[o] for o in orders], 2)          # [B, R, K, 2^bits, D]
    bits = blocks.shape[3].bit_length() - 1
    return ops.select_candidates(blocks, next_codes, bits)
