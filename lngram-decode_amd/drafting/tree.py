"""Draft-tree structure, verification gather and greedy acceptance (``drafting/tree.py`` of the
reference: ``TreeSpec :37-51``, ``default_tree :54-57``, ``chain_tree :60-61``, structure
helpers ``:65-127``, ``tree_route_tokens :130-136``, ``tree_accept :205-220``,
``draft_tree :243-257``).

A tree is ``parent`` (node 0 = root = the pending token, ``parent[0] = -1``, ``parent[i] < i``)
plus ``rank`` (node i takes its parent's rank-th drafted candidate).  Structure helpers are
host integer bookkeeping over at most a few dozen nodes; the row gather and the acceptance run
on the GPU (``lng_route_tokens`` / ``lng_tree_accept``).  With a ``GpuDrafter``,
``draft_tree`` runs every parent of one depth in one batched readout.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor

from lngram_hip import ops


@dataclass(frozen=True)
class TreeSpec:
    parent: tuple
    rank: tuple

    def __post_init__(self):
        if len(self.parent) != len(self.rank) or not self.parent or self.parent[0] != -1:
            raise ValueError("parent[0] must be -1 and parent/rank have equal length")
        for i, p in enumerate(self.parent[1:], 1):
            if not 0 <= p < i:
                raise ValueError(f"node {i}: parent {p} must precede it")

    @property
    def n(self) -> int:
        return len(self.parent)


def default_tree() -> TreeSpec:
    """8 nodes: top-1 chain of depth 4, the runner-up at the first position and its top-1 child,
    the runner-up at the second position."""
    return TreeSpec((-1, 0, 1, 2, 3, 0, 5, 1), (0, 0, 0, 0, 0, 1, 0, 1))


def tree16() -> TreeSpec:
    """16 nodes, depth 4: the top-1 chain, a full runner-up chain from the root, runner-ups at
    depths 2-4 and a third candidate at the root (10 parent readouts in 4 depths, top-3)."""
    return TreeSpec((-1, 0, 1, 2, 3, 0, 5, 6, 7, 1, 9, 10, 2, 12, 3, 0),
                    (0, 0, 0, 0, 0, 1, 0, 0, 0, 1, 0, 0, 1, 0, 1, 2))


def chain_tree(n: int) -> TreeSpec:
    return TreeSpec((-1,) + tuple(range(n - 1)), (0,) * n)


# ---------------------------------------------------------------------- structure
def tree_depths(parent) -> list:
    d: list = []
    for p in parent:
        d.append(0 if p < 0 else d[p] + 1)
    return d


def tree_path(parent, i: int) -> list:
    """Root .. i."""
    out = []
    while i >= 0:
        out.append(i)
        i = parent[i]
    return out[::-1]


def tree_positions(parent, L: int = 0, device=None) -> Tensor:
    return L + torch.tensor(tree_depths(parent), dtype=torch.long, device=device)


def tree_attention_mask(parent, L: int = 0, device=None) -> Tensor:
    """bool [n, L + n]: every cached position, plus ancestors and self."""
    n = len(parent)
    m = torch.zeros(n, L + n, dtype=torch.bool)
    m[:, :L] = True
    for i in range(n):
        for a in tree_path(parent, i):
            m[i, L + a] = True
    return m.to(device) if device is not None else m


def tree_slots(parent, L: int, back: int) -> tuple[Tensor, Tensor]:
    """Slots [n, back+1] (oldest first) of each node's ``back`` predecessors along its ancestors,
    then the ``L`` positions before the root; slot L + a = node a.  Validity alongside."""
    n = len(parent)
    idx = torch.zeros(n, back + 1, dtype=torch.long)
    ok = torch.zeros(n, back + 1, dtype=torch.bool)
    for i in range(n):
        path = tree_path(parent, i)
        for j in range(back + 1):
            s = L + path[len(path) - 1 - j] if j < len(path) else L - (j - len(path) + 1)
            if s >= 0:
                idx[i, back - j], ok[i, back - j] = s, True
    return idx, ok


def tree_ngram_codes(parent_idx, codes: Tensor, history: Tensor | None = None, hist: int = 2):
    """Each node's n-gram code window from its ancestors, then ``history`` (oldest first):
    (ctx [B, n, hist + 1, R], valid [n, hist + 1]); invalid slots hold 0."""
    b, n, r = codes.shape
    h = 0 if history is None else history.shape[1]
    allc = codes if history is None else torch.cat((history.to(codes.dtype), codes), 1)
    idx, ok = tree_slots(parent_idx, h, hist)
    idx, ok = idx.to(codes.device), ok.to(codes.device)
    ctx = allc[:, idx.clamp_min(0)] * ok[None, :, :, None].to(codes.dtype)
    return ctx, ok


def tree_route_tokens(m, ctx: Tensor, valid: Tensor) -> Tensor:
    """Route tokens [B, n, R, Dt] of the n-grams ending at each node: the v2 lookup over the
    windows, invalid slots as their own segment (zero rows), last position only."""
    b, n, w, r = ctx.shape
    seg = valid.to(torch.int32)[None].expand(b, n, w).reshape(b * n, w)
    rt = m._lookup_route_chunk(ctx.reshape(b * n, w, r), None, 0, m.num_routes, seg, None, target_length=1)
    return rt[:, -1].reshape(b, n, r, -1)


# ---------------------------------------------------------------------- acceptance / drafting
def tree_accept(parent, node_tokens, argmax) -> tuple[list, list]:
    """Longest root-to-node path whose tokens equal the verifier's argmax at their parent (first
    matching child in index order) -> (path nodes incl. root, accepted tokens + the verifier's
    token after the path).  Runs ``lng_tree_accept`` on the GPU; device tensors stay there until
    the two small results are read back."""
    dev = argmax.device if isinstance(argmax, Tensor) and argmax.is_cuda else torch.device("cuda")
    par = torch.as_tensor(list(parent), dtype=torch.int32, device=dev)
    nt = torch.as_tensor(node_tokens, dtype=torch.int64).to(dev)
    am = torch.as_tensor(argmax, dtype=torch.int64).to(dev)
    path, plen, new = ops.tree_accept(par, nt, am)
    k = int(plen.item())
    return path[:k].tolist(), new[:k].tolist()


def draft_tree(drafter, spec: TreeSpec) -> list:
    """Node tokens: root = the drafter's last committed token; node i = rank[i]-th candidate after
    its parent's path (top-1 when there is no such candidate).  A drafter with a batched
    ``draft_tree`` runs it; any other drafter gets one ``draft(1, path, topk)`` per parent."""
    if hasattr(drafter, "draft_tree"):
        return drafter.draft_tree(spec)
    k = max(spec.rank) + 1
    toks = [drafter.tokens[-1]]
    cache: dict = {}
    for i in range(1, spec.n):
        p = spec.parent[i]
        if p not in cache:
            hyp = [toks[a] for a in tree_path(spec.parent, p)[1:]]
            cache[p] = drafter.draft(1, hyp, topk=k).topk_ids[0]
        ids = cache[p]
        t = int(ids[spec.rank[i]])
        toks.append(t if t >= 0 else int(ids[0]))
    return toks
