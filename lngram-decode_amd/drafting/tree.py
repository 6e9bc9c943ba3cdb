"""Draft trees: structure, verification gather and greedy acceptance, behind the names of the
reference's ``drafting/tree.py`` (``TreeSpec :37-51``, ``default_tree :54-57``, ``chain_tree
:60-61``, structure helpers ``:65-127``, ``tree_route_tokens :130-136``, ``tree_accept :205-220``,
``draft_tree :243-257``).

A tree is ``parent`` (node 0 is the root, the pending token; ``parent[0] = -1`` and every other
parent precedes its child) plus ``rank`` (node i takes its parent's rank-th drafted candidate).

Every structure helper here is read off one table, the ancestry matrix ``anc[i, j]`` = "node j
lies on the path from the root to node i" (i included).  Because parents precede children, a
node's row is its parent's row plus itself, the ancestors of i in increasing index order are its
path from the root, the row sum is its depth + 1, and the matrix itself is the tree part of the
verification attention mask.  The code window of a node (the slots an n-gram ending at the node
reads) walks up that path and then back into the cached history.  The row gather and the
acceptance run on the GPU.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch
from torch import Tensor

from lngram_hip import ops


@dataclass(frozen=True)
class TreeSpec:
    """``parent`` / ``rank`` tuples; the constructor rejects a root other than node 0, a parent
    that does not precede its child and mismatched lengths."""

    parent: tuple
    rank: tuple

    def __post_init__(self):
        par = list(self.parent)
        if not par or len(par) != len(self.rank) or par[0] != -1:
            raise ValueError("parent[0] must be -1 and parent/rank have equal length")
        bad = [i for i, p in enumerate(par) if i and not 0 <= p < i]
        if bad:
            raise ValueError(f"node {bad[0]}: parent {par[bad[0]]} must precede it")

    @property
    def n(self) -> int:
        return len(self.parent)


def chain_tree(n: int) -> TreeSpec:
    """A single top-1 chain of ``n`` nodes (speculative chain drafting as a tree)."""
    return TreeSpec(tuple(i - 1 for i in range(n)), tuple([0] * n))


def default_tree() -> TreeSpec:
    """8 nodes: a top-1 chain of depth 4 from the root, the root's runner-up with its top-1 child,
    and the runner-up after the first chain node."""
    return TreeSpec((-1, 0, 1, 2, 3, 0, 5, 1), (0, 0, 0, 0, 0, 1, 0, 1))


def tree16() -> TreeSpec:
    """16 nodes, depth 4: the top-1 chain, a full runner-up chain from the root, runner-ups at
    depths 2-4 and a third candidate at the root (10 parent readouts in 4 depths, top-3)."""
    return TreeSpec((-1, 0, 1, 2, 3, 0, 5, 6, 7, 1, 9, 10, 2, 12, 3, 0),
                    (0, 0, 0, 0, 0, 1, 0, 0, 0, 1, 0, 0, 1, 0, 1, 2))


# ---------------------------------------------------------------------- structure
def ancestry(parent) -> np.ndarray:
    """bool ``[n, n]``: ``anc[i, j]`` iff node j is on the root..i path (node i included)."""
    par = np.asarray(parent, dtype=np.int64)
    anc = np.eye(len(par), dtype=bool)
    for i in np.flatnonzero(par >= 0):
        anc[i] |= anc[par[i]]
    return anc


def tree_depths(parent) -> list:
    """Depth of every node (root 0)."""
    return (ancestry(parent).sum(1) - 1).tolist()


def tree_path(parent, i: int) -> list:
    """Nodes from the root to ``i``."""
    return np.flatnonzero(ancestry(parent)[i]).tolist()


def tree_positions(parent, L: int = 0, device=None) -> Tensor:
    """Sequence position of every node when the root sits at position ``L``."""
    return torch.as_tensor(ancestry(parent).sum(1) - 1 + L, dtype=torch.long, device=device)


def tree_attention_mask(parent, L: int = 0, device=None) -> Tensor:
    """bool ``[n, L + n]``: every node sees the ``L`` cached positions, its ancestors and itself."""
    anc = torch.from_numpy(ancestry(parent))
    mask = torch.cat((torch.ones(anc.shape[0], L, dtype=torch.bool), anc), 1)
    return mask.to(device) if device is not None else mask


def tree_slots(parent, L: int, back: int) -> tuple[Tensor, Tensor]:
    """The code window of every node: slots ``[n, back + 1]``, oldest first, ending at the node.
    Slot ``L + a`` is node a and slots below ``L`` are the cached history (the root's predecessor
    is ``L - 1``); a window that reaches before position 0 holds invalid slots (``ok`` False,
    index 0)."""
    anc = ancestry(parent)
    n = anc.shape[0]
    depth = anc.sum(1) - 1
    # up[i, k] = the ancestor of node i at depth k (k <= depth[i])
    up = np.zeros((n, n), dtype=np.int64)
    for i in range(n):
        path = np.flatnonzero(anc[i])
        up[i, :len(path)] = path
    dist = back - np.arange(back + 1)[None, :]                 # steps back from the node
    in_tree = dist <= depth[:, None]
    k = np.clip(depth[:, None] - dist, 0, None)
    slots = np.where(in_tree, L + np.take_along_axis(up, k, 1), L - (dist - depth[:, None]))
    ok = slots >= 0
    return torch.from_numpy(np.where(ok, slots, 0)), torch.from_numpy(ok)


def tree_ngram_codes(parent_idx, codes: Tensor, history: Tensor | None = None, hist: int = 2):
    """Every node's code window along its ancestors, then ``history`` (oldest first):
    ``(ctx [B, n, hist + 1, R], valid [n, hist + 1])``, invalid slots zero."""
    h = 0 if history is None else history.shape[1]
    seq = codes if history is None else torch.cat((history.to(codes.dtype), codes), 1)
    idx, ok = tree_slots(parent_idx, h, hist)
    idx, ok = idx.to(codes.device), ok.to(codes.device)
    ctx = torch.index_select(seq, 1, idx.reshape(-1)).view(codes.shape[0], *idx.shape, codes.shape[2])
    return ctx * ok[None, :, :, None].to(codes.dtype), ok


def tree_route_tokens(m, ctx: Tensor, valid: Tensor) -> Tensor:
    """Route tokens ``[B, n, R, Dt]`` of the n-grams ending at each node (the node windows of
    :func:`tree_ngram_codes`; an n-gram that reaches an invalid slot reads the zero row)."""
    from .drafters import window_route_tokens

    b, n, w, r = ctx.shape
    real = valid.to(ctx.device)[None].expand(b, n, w).reshape(b * n, w)
    return window_route_tokens(m, ctx.reshape(b * n, w, r), real).view(b, n, r, -1)


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
    """Node tokens: the root is the drafter's last committed token; node i is the rank[i]-th
    candidate after its parent's path (the top-1 when there is no such candidate).  A drafter
    with its own batched ``draft_tree`` runs that; any other drafter is asked once per parent
    (``draft(1, path, topk)``), parents in index order."""
    if hasattr(drafter, "draft_tree"):
        return drafter.draft_tree(spec)
    anc = ancestry(spec.parent)
    k = max(spec.rank) + 1
    toks = np.full(spec.n, -1, dtype=np.int64)
    toks[0] = drafter.tokens[-1]
    cand: dict = {}
    for i in range(1, spec.n):
        p = spec.parent[i]
        if p not in cand:
            path = np.flatnonzero(anc[p])[1:]
            cand[p] = drafter.draft(1, [int(x) for x in toks[path]], topk=k).topk_ids[0]
        pick = int(cand[p][spec.rank[i]])
        toks[i] = pick if pick >= 0 else int(cand[p][0])
    return toks.tolist()
