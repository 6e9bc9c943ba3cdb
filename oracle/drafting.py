"""Oracle: CPU restatement of the self-drafting readers (test infrastructure only).

Restates, in fp64 by default (``dtype=torch.float32`` gives the reference's own fp32
arithmetic):

- the per-token drafter ``RefDrafter`` (``drafting/cpu_drafter.py:76-289``): router codes
  from ``concat(RMSNorm(E[x_{t-1}] or start), RMSNorm(E[x_t])[, s_t])``, v2 n-gram rows,
  ``DraftReadout.hidden`` (memory RMSNorm -> KV projection -> sink softmax over routes ->
  ``W_o`` -> RMSNorm), logits against the tied embedding, top-k by (logit desc, index asc);
  stateful commit / draft / truncate / trace.  Scoring is over the full vocabulary, or over the
  count-sketch shortlist of ``cpu_drafter.py:179-206`` when the bundle carries sketches and a
  positive ``shortlist_cap`` (``sketch_shortlist`` below).
- code-keyed online counts (``OnlineCounts.mix``, ``drafting/drafters.py:117-142``), applied
  to the drafter's softmax when ``online=True``;
- the tree structure and verification helpers of ``drafting/tree.py:37-136, :205-257``.

Parameters come as a bundle-style ``config`` dict (keys of ``bundle_config``,
``drafting/export_drafter.py:212-215``) and a ``tensors`` dict keyed like the bundle arrays
(``embedding``, ``table_<n>``, ``mem_norm``, ``kv_proj``, ``router``, ``router_prev_norm``,
``router_cur_norm``, ``router_start``, ``ssm_norm``/``ssm_w_in``/``ssm_decay``, ``q_norm``,
``w_q``, ``w_sq``, ``w_o``, ``out_norm``).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import memory as om


def _rms(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    # cpu_drafter._rms (drafting/cpu_drafter.py:64-65)
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def top_order(logits: torch.Tensor, k: int) -> torch.Tensor:
    """Indices of the ``k`` largest entries ordered by (value desc, index asc)
    (``drafter.cpp:547-556``; the stable descending sort of ``cpu_drafter.py:263``)."""
    return torch.sort(logits, descending=True, stable=True).indices[:k]


@dataclass(frozen=True)
class _Cursor:
    t: int
    tok: int
    s: torch.Tensor | None
    hist: tuple  # codes (np.uint8 [R]) of the last max(ngrams) positions, oldest first


@dataclass
class DraftOut:
    """``DraftOut`` (``cpu_drafter.py:51-61``)."""

    tokens: list
    topk_ids: np.ndarray
    topk_logits: np.ndarray
    codes: np.ndarray

    @property
    def runner_up(self) -> int:
        return int(self.topk_ids[0, 1]) if self.topk_ids.shape[1] > 1 else -1


class DrafterOracle:
    """``RefDrafter`` (``cpu_drafter.py:76-289``) in ``dtype``.

    ``online=True`` mixes the draft softmax with code-keyed online counts over the committed
    (row at t, token t+1) pairs (``drafters.py:117-142``, ``:193-201``); the ranking is then by
    the mixed probability and ``topk_logits`` holds its natural log.
    """

    name = "oracle"

    def __init__(self, config: dict, tensors: dict, topk: int = 3, dtype=torch.float64, online: bool = False,
                 kappa: float = 1.0, shortlist_cap: int | None = None):
        c = self.cfg = dict(config)
        self.dtype = dtype
        self.topk = int(topk)
        self.online, self.kappa = bool(online), float(kappa)
        self.ngrams = [int(n) for n in c["ngrams"]]
        self.maxn = max(self.ngrams)
        self.R, self.bits, self.V = int(c["routes"]), int(c["bits"]), int(c["vocab"])
        self.kv, self.hd, self.G = int(c["kv_heads"]), int(c["head_dim"]), int(c["groups"])
        t = {k: (v.to(dtype) if v.is_floating_point() else v) for k, v in tensors.items()}
        self.E = t["embedding"]
        self.tables = {n: t[f"table_{n}"] for n in self.ngrams}
        self.mem_norm, self.kv_proj, self.router = t["mem_norm"], t["kv_proj"], t["router"]
        self.prev_norm, self.cur_norm, self.start = t["router_prev_norm"], t["router_cur_norm"], t["router_start"]
        self.has_ssm = "ssm_w_in" in t
        if self.has_ssm:
            self.ssm_norm, self.ssm_w_in, self.ssm_a = t["ssm_norm"], t["ssm_w_in"], t["ssm_decay"]
        self.router_ssm = c["router_kind"] == "embed2_ssm"
        self.q_norm, self.w_q, self.w_o, self.out_norm = t["q_norm"], t["w_q"], t["w_o"], t["out_norm"]
        self.w_sq = t.get("w_sq")
        self.shifts = torch.arange(self.bits, dtype=torch.int32)
        # count sketches (cpu_drafter.py:99-103): ids / counts per order, fallback tokens, cap
        self.sk_ids = {n: np.asarray(t[f"sketch_ids_{n}"]).astype(np.int64) for n in self.ngrams
                       if f"sketch_ids_{n}" in t}
        self.sk_cnt = {n: np.asarray(t[f"sketch_counts_{n}"]).astype(np.int64) for n in self.sk_ids}
        fb = t.get("fallback")
        self.fallback = [] if fb is None else [int(x) for x in np.asarray(fb).ravel()]
        self.cap = int(c.get("shortlist_cap", 0)) if shortlist_cap is None else int(shortlist_cap)
        if self.online and self.cap > 0 and self.sk_ids:
            raise ValueError("online counts mix a full-vocabulary softmax; the shortlist drafter has none")
        self.reset()

    # ------------------------------------------------------------------ state (cpu_drafter.py:110-144)
    def reset(self) -> None:
        self._tokens: list = []
        self._codes: list = []
        self._ssm: list = []

    @property
    def length(self) -> int:
        return len(self._tokens)

    @property
    def tokens(self) -> list:
        return list(self._tokens)

    def committed_codes(self) -> np.ndarray:
        return np.stack(self._codes) if self._codes else np.zeros((0, self.R), np.uint8)

    def truncate(self, length: int) -> None:
        if not 0 <= length <= self.length:
            raise ValueError(f"cannot truncate to {length} (length {self.length})")
        del self._tokens[length:], self._codes[length:], self._ssm[length:]

    def commit(self, tokens, codes=None) -> None:
        cur = self._cursor()
        for i, tok in enumerate(tokens):
            cur = self._advance(cur, int(tok), None if codes is None else np.asarray(codes[i], np.uint8))
            self._tokens.append(int(tok))
            self._codes.append(cur.hist[-1])
            self._ssm.append(cur.s)

    def _cursor(self) -> _Cursor:
        n = self.length
        if n == 0:
            return _Cursor(-1, -1, None, ())
        return _Cursor(n - 1, self._tokens[-1], self._ssm[-1], tuple(self._codes[max(0, n - self.maxn):]))

    # ------------------------------------------------------------------ per token (cpu_drafter.py:147-177)
    def router_features(self, prev_tok: int, tok: int, s: torch.Tensor | None) -> torch.Tensor:
        e = self.E[tok]
        ep = self.E[prev_tok] if prev_tok >= 0 else self.start
        eps = self.cfg["router_eps"]
        parts = [_rms(ep, self.prev_norm, eps), _rms(e, self.cur_norm, eps)]
        if self.router_ssm:
            parts.append(s)
        return torch.cat(parts)

    def router_logits(self, prev_tok: int, tok: int, s: torch.Tensor | None) -> torch.Tensor:
        return self.router @ self.router_features(prev_tok, tok, s)

    def _advance(self, cur: _Cursor, tok: int, code: np.ndarray | None = None) -> _Cursor:
        e = self.E[tok]
        s = None
        if self.has_ssm:
            u = self.ssm_w_in @ _rms(e, self.ssm_norm, self.cfg["ssm_eps"])
            prev = cur.s if cur.s is not None else torch.zeros_like(u)
            s = self.ssm_a * prev + (1 - self.ssm_a) * u
        if code is None:
            logits = self.router_logits(cur.tok if cur.t >= 0 else -1, tok, s)
            bits = (logits > 0).view(self.R, self.bits).to(torch.int32)
            code = (bits << self.shifts).sum(-1).to(torch.uint8).numpy()
        return _Cursor(cur.t + 1, tok, s, (cur.hist + (code,))[-self.maxn:])

    def rows(self, cur: _Cursor) -> dict:
        """Global rows per order at the cursor (``cpu_drafter.py:166-177``), None before n-1."""
        out = {}
        r = np.arange(self.R, dtype=np.int64)
        for n in self.ngrams:
            if cur.t < n - 1:
                out[n] = None
                continue
            addr = np.zeros(self.R, np.int64)
            for k in range(n):
                addr |= cur.hist[len(cur.hist) - n + k].astype(np.int64) << (k * self.bits)
            out[n] = r * (1 << self.bits) ** n + addr
        return out

    # ------------------------------------------------------------------ readout (cpu_drafter.py:208-244)
    def hidden(self, cur: _Cursor, rows: dict | None = None) -> torch.Tensor:
        rows = self.rows(cur) if rows is None else rows
        c = self.cfg
        mem_dim = int(c["mem_dim"])
        parts = []
        for n in self.ngrams:
            if rows[n] is None:
                parts.append(torch.zeros(self.R, mem_dim, dtype=self.dtype))
            else:
                parts.append(self.tables[n][torch.from_numpy(rows[n])])
        tok = torch.cat(parts, -1)
        kv = _rms(tok, self.mem_norm, c["mem_eps"]) @ self.kv_proj.T
        kh = self.kv * self.hd
        key = kv[:, :kh].reshape(self.R, self.kv, self.hd).transpose(0, 1)
        val = kv[:, kh:].reshape(self.R, self.kv, self.hd).transpose(0, 1)
        e = self.E[cur.tok]
        q = self.w_q @ _rms(e, self.q_norm, c["draft_eps"])
        if self.w_sq is not None:
            q = q + self.w_sq @ cur.s
        q = q.view(self.kv, self.G, self.hd)
        scores = (q @ key.transpose(-1, -2)) * c["softmax_scale"]
        probs = om.sink_probabilities(scores, float(c["sink_logit"]))
        out = (probs @ val).reshape(-1)
        return _rms(self.w_o @ out, self.out_norm, c["draft_eps"])

    def logits(self, cur: _Cursor) -> torch.Tensor:
        return self.E @ self.hidden(cur)

    # ------------------------------------------------------------------ shortlist (cpu_drafter.py:179-206)
    def shortlist(self, rows: dict) -> list | None:
        """The shortlist at the rows of one position, or None for full-vocabulary scoring."""
        if self.cap <= 0 or not self.sk_ids:
            return None
        return sketch_shortlist(self.sk_ids, self.sk_cnt, self.fallback, rows, self.cap)

    def readout(self, cur: _Cursor, full: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
        """(candidate token ids, logits) at the cursor (``cpu_drafter.py:238-244``): the shortlist
        when there is one (and ``full`` is off), else the whole vocabulary."""
        rows = self.rows(cur)
        h = self.hidden(cur, rows)
        sl = None if full else self.shortlist(rows)
        if sl is None:
            return torch.arange(self.V), self.E @ h
        ids = torch.tensor(sl, dtype=torch.long)
        return ids, self.E[ids] @ h

    # ------------------------------------------------------------------ online counts (drafters.py:117-142)
    def online_mix(self, p: torch.Tensor, cur: _Cursor, n_pairs: int) -> torch.Tensor:
        """``OnlineCounts.mix`` for one query at the cursor, keys = the first ``n_pairs``
        committed (row at t, token t+1) pairs."""
        if n_pairs <= 0:
            return p
        codes = self.committed_codes()[: n_pairs + 1]
        nxt = torch.tensor(self._tokens[1: n_pairs + 1], dtype=torch.long)
        q = self.rows(cur)
        w = torch.zeros(n_pairs, dtype=p.dtype)
        for n in self.ngrams:
            if q[n] is None:
                continue
            keys = seq_rows(codes[None], n, self.bits)[0, :n_pairs]        # [n_pairs, R]
            w += torch.from_numpy(((keys == q[n][None]) & (q[n][None] >= 0)).sum(-1)).to(p.dtype)
        tot = w.sum()
        sc = torch.zeros(self.V, dtype=p.dtype).scatter_add_(0, nxt, w)
        n_eff = tot / (self.R * len(self.ngrams))
        lam = n_eff / (n_eff + self.kappa)
        return (1 - lam) * p + lam * sc / tot.clamp_min(1e-9)

    def distribution(self, cur: _Cursor, n_pairs: int) -> torch.Tensor:
        """Ranking scores of the next token: logits, or log of the online-mixed softmax."""
        lg = self.logits(cur)
        if not self.online:
            return lg
        return torch.log(self.online_mix(torch.softmax(lg, -1), cur, n_pairs))

    # ------------------------------------------------------------------ API (cpu_drafter.py:247-289)
    def draft(self, gamma: int, hyp=(), topk: int | None = None, last_codes: bool = False) -> DraftOut:
        k = int(topk or self.topk)
        cur = self._cursor()
        if cur.t < 0 and not len(hyp):
            raise ValueError("draft needs at least one committed or hypothetical token")
        n_pairs = max(self.length - 1, 0)
        codes = []
        for tok in hyp:
            cur = self._advance(cur, int(tok))
            codes.append(cur.hist[-1])
        ids = np.full((gamma, k), -1, np.int64)
        lg = np.full((gamma, k), -np.inf, np.float32)
        toks = []
        for i in range(gamma):
            if self.online:
                cand, scores = torch.arange(self.V), self.distribution(cur, n_pairs)
            else:
                cand, scores = self.readout(cur)
            order = top_order(scores, k)
            ids[i, :len(order)] = cand[order].numpy()
            lg[i, :len(order)] = scores[order].numpy()
            toks.append(int(ids[i, 0]))
            if i + 1 < gamma or last_codes:
                cur = self._advance(cur, toks[-1])
                codes.append(cur.hist[-1])
        return DraftOut(toks, ids, lg, np.stack(codes) if codes else np.zeros((0, self.R), np.uint8))

    def trace(self, tokens, codes=None) -> tuple[np.ndarray, np.ndarray]:
        """Teacher-forced pass from an empty state (full vocab): (codes [T, R], scores [T, V])."""
        tokens = [int(x) for x in tokens]
        n = len(tokens)
        out_c = np.zeros((n, self.R), np.uint8)
        out_l = np.zeros((n, self.V), np.float64)
        saved = (self._tokens, self._codes, self._ssm)
        self.reset()
        try:
            cur = _Cursor(-1, -1, None, ())
            for t, tok in enumerate(tokens):
                cur = self._advance(cur, tok, None if codes is None else np.asarray(codes[t], np.uint8))
                self._tokens.append(tok)
                self._codes.append(cur.hist[-1])
                self._ssm.append(cur.s)
                out_c[t] = cur.hist[-1]
                out_l[t] = self.distribution(cur, t).numpy()
        finally:
            self._tokens, self._codes, self._ssm = saved
        return out_c, out_l


    def trace_readout(self, tokens, codes=None, full: bool = False):
        """``RefDrafter.trace`` (``cpu_drafter.py:272-289``): per position (codes [T, R], candidate ids
        [T, S] (-1 pad), logits [T, S] (-inf pad)), S = vocab if ``full`` or no shortlist, else cap;
        a position whose shortlist is empty scores the whole vocabulary, cut to S."""
        tokens = [int(x) for x in tokens]
        full_vocab = full or self.cap <= 0 or not self.sk_ids
        s_dim = self.V if full_vocab else self.cap
        n = len(tokens)
        out_c = np.zeros((n, self.R), np.uint8)
        out_i = np.full((n, s_dim), -1, np.int64)
        out_l = np.full((n, s_dim), -np.inf, np.float64)
        cur = _Cursor(-1, -1, None, ())
        for t, tok in enumerate(tokens):
            cur = self._advance(cur, tok, None if codes is None else np.asarray(codes[t], np.uint8))
            out_c[t] = cur.hist[-1]
            ids, lg = self.readout(cur, full)
            m = min(len(ids), s_dim)
            out_i[t, :m], out_l[t, :m] = ids[:m].numpy(), lg[:m].double().numpy()
        return out_c, out_i, out_l


def sketch_shortlist(sk_ids: dict, sk_cnt: dict, fallback, rows: dict, cap: int) -> list | None:
    """The deterministic shortlist of ``RefDrafter._shortlist`` (``cpu_drafter.py:179-206``,
    ``drafter.cpp:438-474``): the counts of every sketch slot (count > 0) of the position's rows,
    over orders and routes, summed per token; tokens ordered by (total desc, id asc) and cut to
    ``cap``; then the ``fallback`` tokens not yet present, in their order, up to ``cap``.  None
    when that leaves it empty.  ``rows``: order -> int64 [R] global rows, or None before n-1."""
    total: dict = {}
    for n, r in rows.items():
        if r is None or n not in sk_ids:
            continue
        for tok, cnt in zip(sk_ids[n][r].ravel().tolist(), sk_cnt[n][r].ravel().tolist()):
            if cnt > 0:
                total[tok] = total.get(tok, 0) + cnt
    out = sorted(total, key=lambda v: (-total[v], v))[:cap]
    seen = set(out)
    for f in fallback:
        if len(out) >= cap:
            break
        if f not in seen:
            out.append(f)
            seen.add(f)
    return out or None


# ----------------------------------------------------------------------------- rows helpers
def seq_rows(codes, order: int, bits: int) -> np.ndarray:
    """``seq_rows`` (``drafting/build_sketches.py:186-197``): rows [B, T, R] of the n-grams
    ending at each t, -1 for t < order-1 (oldest code least significant)."""
    c = np.asarray(codes).astype(np.int64)
    b, t, r = c.shape
    out = np.full((b, t, r), -1, np.int64)
    if t >= order:
        addr = c[:, : t - order + 1].copy()
        for e in range(1, order):
            addr |= c[:, e: e + t - order + 1] << (e * bits)
        out[:, order - 1:] = np.arange(r, dtype=np.int64) * (1 << (bits * order)) + addr
    return out


def window_rows(win, real, order: int, bits: int) -> np.ndarray:
    """``window_rows`` (``drafting/drafters.py:99-107``): rows [N, R] of the n-gram ending at
    the window's last position, -1 if any of its positions is not real."""
    win = np.asarray(win).astype(np.int64)
    real = np.asarray(real, bool)
    n, w, r = win.shape
    c = win[:, w - order:]
    addr = c[:, 0].copy()
    for e in range(1, order):
        addr |= c[:, e] << (e * bits)
    rows = np.arange(r, dtype=np.int64) * (1 << (bits * order)) + addr
    return np.where(real[:, w - order:].all(1, keepdims=True), rows, -1)


def online_counts_mix(p, codes, x, orders, bits: int, win, real, deadline, kappa: float = 1.0):
    """``OnlineCounts(codes, x).mix(p, win, real, deadline)`` (``drafters.py:117-142``) in fp64:
    keys = rows of the pairs (t, x[t+1]) for t = 0 .. T-2, only t <= deadline[j] counts."""
    p = torch.as_tensor(p, dtype=torch.float64)
    codes = np.asarray(codes)
    x = np.asarray(x, np.int64)
    n_rows = p.shape[0]
    t_len = len(x) - 1
    routes = codes.shape[1]
    ok_t = np.arange(t_len)[None] <= np.asarray(deadline)[:, None]
    w = np.zeros((n_rows, t_len))
    for n in orders:
        keys = seq_rows(codes[None], n, bits)[0, :-1]
        q = window_rows(win, real, n, bits)
        w += ((keys[None] == q[:, None]) & (q[:, None] >= 0)).sum(-1)
    w = torch.from_numpy(w * ok_t)
    tot = w.sum(1, keepdim=True)
    sc = torch.zeros(n_rows, p.shape[1], dtype=torch.float64).scatter_add_(
        1, torch.from_numpy(x[1:])[None].expand(n_rows, -1), w)
    n_eff = tot / (routes * len(orders))
    lam = n_eff / (n_eff + kappa)
    return (1 - lam) * p + lam * sc / tot.clamp_min(1e-9)


# ----------------------------------------------------------------------------- tree (tree.py:37-136, :205-257)
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


def tree_depths(parent) -> list:
    d = []
    for p in parent:
        d.append(0 if p < 0 else d[p] + 1)
    return d


def tree_path(parent, i: int) -> list:
    out = []
    while i >= 0:
        out.append(i)
        i = parent[i]
    return out[::-1]


def tree_attention_mask(parent, L: int = 0) -> np.ndarray:
    n = len(parent)
    m = np.zeros((n, L + n), bool)
    m[:, :L] = True
    for i in range(n):
        for a in tree_path(parent, i):
            m[i, L + a] = True
    return m


def tree_slots(parent, L: int, back: int) -> tuple[np.ndarray, np.ndarray]:
    """Slots [n, back+1] (oldest first) of each node's predecessors along its ancestors, then
    the L positions before the root (``tree.py:96-111``)."""
    n = len(parent)
    idx = np.zeros((n, back + 1), np.int64)
    ok = np.zeros((n, back + 1), bool)
    for i in range(n):
        path = tree_path(parent, i)
        for j in range(back + 1):
            s = L + path[len(path) - 1 - j] if j < len(path) else L - (j - len(path) + 1)
            if s >= 0:
                idx[i, back - j], ok[i, back - j] = s, True
    return idx, ok


def tree_ngram_codes(parent, codes, history=None, hist: int = 2):
    """``tree_ngram_codes`` (``tree.py:114-127``): ctx [B, n, hist+1, R], valid [n, hist+1]."""
    codes = np.asarray(codes)
    h = 0 if history is None else np.asarray(history).shape[1]
    allc = codes if history is None else np.concatenate((np.asarray(history).astype(codes.dtype), codes), 1)
    idx, ok = tree_slots(parent, h, hist)
    ctx = allc[:, idx] * ok[None, :, :, None].astype(codes.dtype)
    return ctx, ok


def tree_route_tokens(tables: dict, orders, bits: int, ctx, valid) -> torch.Tensor:
    """``tree_route_tokens`` (``tree.py:130-136``): [B, n, R, Dt], invalid window slots form
    their own segment (zero rows for n-grams reaching them)."""
    b, n, w, r = ctx.shape
    seg = np.broadcast_to(np.asarray(valid, np.int32)[None], (b, n, w)).reshape(b * n, w)
    rt = om.route_tokens(tables, ctx.reshape(b * n, w, r), orders, bits, 0, r, segment_ids=seg)
    return rt[:, -1].reshape(b, n, r, -1)


def tree_accept(parent, node_tokens, argmax) -> tuple[list, list]:
    """``tree_accept`` (``tree.py:205-220``)."""
    children: dict = {}
    for i, p in enumerate(parent):
        if p >= 0:
            children.setdefault(p, []).append(i)
    path, cur = [0], 0
    while True:
        nxt = next((c for c in children.get(cur, []) if int(node_tokens[c]) == int(argmax[cur])), None)
        if nxt is None:
            break
        path.append(nxt)
        cur = nxt
    return path, [int(node_tokens[c]) for c in path[1:]] + [int(argmax[cur])]


def draft_tree(drafter, spec: TreeSpec) -> list:
    """``draft_tree`` (``tree.py:243-257``): node i = the rank[i]-th candidate after its
    parent's path (-1 falls back to the top-1)."""
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
