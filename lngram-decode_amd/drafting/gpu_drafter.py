"""MI355X drafter: the stateful drafter API of ``drafting/cpu_drafter.py`` (``RefDrafter`` /
``CppDrafter``: ``reset / length / tokens / committed_codes / truncate / commit / draft /
trace``, ``DraftOut``) with every per-token step on the GPU (``lng_drafter_*`` in
``include/lngram_hip.h``).

Per token, as ``cpu_drafter.py:13-28`` describes: SSM step, router codes from
``concat(RMSNorm(E[x_{t-1}] or start), RMSNorm(E[x_t])[, s_t])``, the v2 n-gram rows, the draft
readout over the shared table (memory norm, KV projection, sink softmax over routes, ``W_o``,
RMSNorm) and logits against the tied embedding, top-k by (logit desc, id asc).  With count
sketches in the bundle and a positive ``shortlist_cap`` the drafts are scored over the sketch
shortlist instead (``cpu_drafter.py:179-206``: sketch tokens of the position's rows by summed
count, padded with the fallback tokens; ``lng_drafter_shortlist``).  With ``online=True``
the draft distribution is mixed with code-keyed online counts over the committed
(row at t, token t+1) pairs (``drafting/drafters.py:117-142``); candidates are then ranked by,
and ``topk_logits`` holds, the log of the mixed probability.

State lives on the device: token ids, route codes and SSM states per committed position, plus
scratch rows for hypothetical positions and draft-tree nodes.  ``draft`` never mutates the
committed state; ``truncate`` is exact rollback.
"""

from __future__ import annotations

import ctypes
import threading

import numpy as np
import torch

from lngram_hip import _lib, ops
from lngram_hip._lib import ROW_NONE, check

from .cpu_drafter import DraftOut
from .export_drafter import Bundle

_TREE_ROWS = 64
_HYP_ROWS = 192
_MAX_K = 8


def _bundle_parts(bundle) -> tuple[dict, dict]:
    if isinstance(bundle, Bundle):
        return dict(bundle.config), bundle.tensors()
    if isinstance(bundle, tuple) and len(bundle) == 2:
        return dict(bundle[0]), dict(bundle[1])
    from .export_drafter import load_bundle

    b = load_bundle(bundle)
    return dict(b.config), b.tensors()


def _dt(t: torch.Tensor) -> int:
    return ops.dtype_code(t.dtype)


class GpuDrafter:
    """Drafter with the reference API, running on ``device`` (a ROCm GPU)."""

    name = "gpu"

    def __init__(self, bundle, topk: int = 3, shortlist_cap: int | None = None, device=None, max_len: int = 4096,
                 online: bool = False, kappa: float = 1.0, tables: bool = True, levels: bool = True):
        c, t = _bundle_parts(bundle)
        self.cfg = c
        # RefDrafter scores a sketch shortlist when the cap is positive and the bundle carries
        # sketches (cpu_drafter.py:102-105, :179-181)
        cap = int(c.get("shortlist_cap", 0) if shortlist_cap is None else shortlist_cap)
        self.cap = cap if cap > 0 and any(f"sketch_ids_{n}" in t for n in c["ngrams"]) else 0
        if self.cap and online:
            raise ValueError("the sketch shortlist and online counts do not combine (RefDrafter scores the "
                             "shortlist without online counts)")
        self.topk = int(topk)
        self.online, self.kappa = bool(online), float(kappa)
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        if dev.type != "cuda":
            raise RuntimeError("GpuDrafter needs a ROCm GPU device; there is no CPU path")
        self.device = dev
        self.ngrams = [int(n) for n in c["ngrams"]]
        self.maxn = max(self.ngrams)
        self.R, self.bits, self.V, self.d = int(c["routes"]), int(c["bits"]), int(c["vocab"]), int(c["d_model"])
        self.kv, self.hd, self.qh = int(c["kv_heads"]), int(c["head_dim"]), int(c["q_heads"])
        self.G = self.qh // self.kv
        self.mem_dim = int(c["mem_dim"])
        self.dt = len(self.ngrams) * self.mem_dim
        self.N = int(c.get("ssm_dim", 0) or 0)
        self.router_ssm = c["router_kind"] == "embed2_ssm"
        self.query_ssm = "w_sq" in t
        has_ssm = "ssm_w_in" in t
        if (self.router_ssm or self.query_ssm) and not has_ssm:
            raise ValueError("drafter reads an SSM state but the bundle has no SSM")
        if not has_ssm:
            self.N = 0
        self.max_len = int(max_len)
        self._lock = threading.Lock()

        def f32(k):
            return t[k].to(dev, torch.float32).contiguous()

        def keep(k):
            x = t[k]
            if x.dtype not in (torch.float32, torch.bfloat16, torch.float16):
                x = x.float()
            return x.to(dev).contiguous()

        self.sketch = self._load_sketch(t, dev) if self.cap else None
        self.emb = keep("embedding")
        self.tables = [keep(f"table_{n}") for n in self.ngrams]
        if len({x.dtype for x in self.tables}) != 1:
            raise ValueError("all n-gram tables must share one dtype")
        self.router = keep("router")
        self.vec = {k: f32(k) for k in ("router_start", "router_prev_norm", "router_cur_norm", "out_norm")}
        if self.N:
            self.vec.update({k: f32(k) for k in ("ssm_norm", "ssm_w_in", "ssm_decay")})
        self._compose(t, dev)
        self.luts = None
        if tables and not (self.router_ssm or self.query_ssm) and self.qh * self.hd <= 256:
            self._build_luts(t, dev)

        rows = self.max_len + _TREE_ROWS + _HYP_ROWS
        self.rows = rows
        self.tree_row0 = self.max_len
        self.hyp_row0 = self.max_len + _TREE_ROWS
        self.tok_d = torch.zeros(rows, dtype=torch.int64, device=dev)
        self.codes_d = torch.zeros(rows, self.R, dtype=torch.uint8, device=dev)
        self.ssm_d = torch.zeros(rows, max(self.N, 1), dtype=torch.float32, device=dev)
        self.len_d = torch.zeros(1, dtype=torch.int32, device=dev)
        # block counters of the kernels that hand partial results to a last block (zero between calls)
        self.sync = torch.zeros(_lib.DR_SYNC_INTS, dtype=torch.int32, device=dev)
        self.D = self._descriptor(self.tok_d, self.codes_d, self.ssm_d, self.len_d, rows)
        self.lib = _lib.load()
        if self.lib.lng_drafter_size() != ctypes.sizeof(_lib.Drafter):
            raise RuntimeError("lng_drafter layout mismatch between the library and its binding")
        nbytes = self.lib.lng_drafter_workspace_bytes(ctypes.byref(self.D), 16, _MAX_K, rows)
        if nbytes == 0:
            raise ValueError("drafter shape outside the kernels' limits")
        self.work = torch.empty(int(nbytes), dtype=torch.uint8, device=dev)
        self.counts = torch.zeros(16, self.V, dtype=torch.int32, device=dev)
        self._graphs: dict = {}          # (parent, rank, route_tokens) -> (captured tree step, out)
        # draft trees of token-only drafters at the SD drafters' shape: the one-launch tree
        # (lng_drafter_tree_levels); trees outside its limits take the per-depth readouts of
        # lng_drafter_tree.  Its workspace keeps a call epoch, so it is zeroed once here.
        self.level_work = None
        self._level_specs: dict = {}
        if levels and self.luts is not None and self.sketch is None:
            lb = self.lib.lng_drafter_tree_levels_workspace(ctypes.byref(self.D))
            if lb:
                self.level_work = torch.zeros(int(lb), dtype=torch.uint8, device=dev)
        self.ids_d = torch.empty(_HYP_ROWS, _MAX_K, dtype=torch.int64, device=dev)
        self.sc_d = torch.empty(_HYP_ROWS, _MAX_K, dtype=torch.float32, device=dev)
        # a draft's results (top-k ids, scores, codes of the drafted rows) leave the device in one
        # copy: packed into a device staging buffer, then copied to pinned host memory
        self._out_bytes = _HYP_ROWS * _MAX_K * 12 + _HYP_ROWS * self.R
        self._out_d = torch.empty(self._out_bytes, dtype=torch.uint8, device=dev)
        self._out_h = torch.empty(self._out_bytes, dtype=torch.uint8, pin_memory=True)
        if self.sketch is not None:
            # full-vocabulary logits and top-k of up to 16 positions (the inputs of lng_drafter_shortlist
            # in trace and of the tree shortlist; chain drafts score only the shortlist)
            self.sl_lg = torch.empty(16, self.V, dtype=torch.float32, device=dev)
            self.sl_fid = torch.empty(16 * _MAX_K, dtype=torch.int64, device=dev)
            self.sl_fsc = torch.empty(16 * _MAX_K, dtype=torch.float32, device=dev)
        self.reset()

    def _load_sketch(self, t: dict, dev) -> _lib.Sketch:
        """Device copies of the bundle's count sketches (ids int32, counts int64) and fallback list,
        and their ``lng_sketch`` descriptor."""

        def host(x) -> np.ndarray:
            return np.asarray(x.cpu() if torch.is_tensor(x) else x)

        S = _lib.Sketch()
        keep = []
        k = None
        for i, n in enumerate(self.ngrams):
            if f"sketch_ids_{n}" not in t:
                continue
            ids, cnt = host(t[f"sketch_ids_{n}"]), host(t[f"sketch_counts_{n}"])
            rows = self.R * (1 << (self.bits * n))
            if ids.ndim != 2 or ids.shape[0] != rows or cnt.shape != ids.shape:
                raise ValueError(f"sketch of order {n} must be [{rows}, K] ids and counts")
            if k is not None and ids.shape[1] != k:
                raise ValueError("every order's sketch must have the same K")
            k = ids.shape[1]
            ids_d = torch.from_numpy(ids.astype(np.int32)).to(dev)
            cnt_d = torch.from_numpy(cnt.astype(np.int64)).to(dev)
            keep += [ids_d, cnt_d]
            S.ids[i], S.counts[i] = ids_d.data_ptr(), cnt_d.data_ptr()
        fb = t.get("fallback")
        fb = np.zeros(0, np.int32) if fb is None else host(fb).ravel()
        if len(fb) > 1024:
            raise ValueError("at most 1024 fallback tokens")
        fb_d = torch.from_numpy(fb.astype(np.int32)).to(dev) if len(fb) else torch.zeros(1, dtype=torch.int32,
                                                                                          device=dev)
        keep.append(fb_d)
        S.k, S.cap, S.fallback, S.n_fallback = int(k), self.cap, fb_d.data_ptr(), len(fb)
        if len(self.ngrams) * self.R * int(k) > 8192 or self.R > 256 or self.cap > 256:
            raise NotImplementedError("the shortlist kernel takes n_orders * R * K <= 8192 sketch slots per "
                                      "position, R <= 256 and a cap <= 256")
        self._sketch_keep = keep
        return S

    # ------------------------------------------------------------------ set-up
    def _compose(self, t: dict, dev) -> None:
        """Precompose the readout's fp32 matrices qk, qks, ov (see ``lng_drafter``)."""
        c = self.cfg
        kh = self.kv * self.hd
        kvp = t["kv_proj"].to(dev, torch.float32)
        mem_norm = t["mem_norm"].to(dev, torch.float32)
        q_norm = t["q_norm"].to(dev, torch.float32)
        w_q = t["w_q"].to(dev, torch.float32)
        w_o = t["w_o"].to(dev, torch.float32)
        scale = float(c["softmax_scale"])
        qk, ov, qks = [], [], []
        w_sq = t["w_sq"].to(dev, torch.float32) if self.query_ssm else None
        for qh in range(self.qh):
            h = qh // self.G
            wk_t = kvp[h * self.hd:(h + 1) * self.hd].t().contiguous()             # [Dt, hd]
            wv = kvp[kh + h * self.hd: kh + (h + 1) * self.hd]                     # [hd, Dt]
            wq_t = w_q[qh * self.hd:(qh + 1) * self.hd].t().contiguous()           # [d, hd]
            qk.append(ops.linear(wk_t, wq_t))                                      # [Dt, d]
            if w_sq is not None:
                qks.append(ops.linear(wk_t, w_sq[qh * self.hd:(qh + 1) * self.hd].t().contiguous()))
            ov.append(ops.linear(w_o[:, qh * self.hd:(qh + 1) * self.hd].contiguous(), wv.t().contiguous()))
        rs = (scale * mem_norm)[:, None]
        self.qk = (torch.cat(qk, 0).view(self.qh, self.dt, self.d) * rs[None] * q_norm[None, None]).reshape(
            self.qh * self.dt, self.d).contiguous()
        self.qks = (torch.cat(qks, 0).view(self.qh, self.dt, -1) * rs[None]).reshape(self.qh * self.dt, -1).contiguous() \
            if qks else None
        self.ov = torch.stack(ov, 1).mul(mem_norm[None, None]).reshape(self.d, self.qh * self.dt).contiguous()

    def _build_luts(self, t: dict, dev) -> None:
        """Per-token tables of the token-only drafter (``lng_drafter.lut_*``), fp32."""
        c = self.cfg
        d, kh = self.d, self.kv * self.hd
        ef = self.emb.float()
        rw = self.router.float()
        ones = torch.ones(d, dtype=torch.float32, device=dev)
        reps = float(c["router_eps"])
        lut = {}
        lut["lut_prev"] = ops.linear(ops.rmsnorm(ef, self.vec["router_prev_norm"], reps), rw[:, :d].contiguous())
        lut["lut_cur"] = ops.linear(ops.rmsnorm(ef, self.vec["router_cur_norm"], reps), rw[:, d:2 * d].contiguous())
        lut["lut_start"] = ops.linear(ops.rmsnorm(self.vec["router_start"][None], self.vec["router_prev_norm"], reps),
                                      rw[:, :d].contiguous())[0].contiguous()
        lut["lut_qk"] = ops.linear(ops.rmsnorm(ef, ones, float(c["draft_eps"])), self.qk)
        w_o_t = t["w_o"].to(dev, torch.float32).t().contiguous()                  # [I, d]
        lut["lut_out"] = ops.linear(ef * self.vec["out_norm"][None], w_o_t)
        if (self.qh * self.hd) % 16 == 0:
            lut["lut_out_pk"] = self._pack_tiles(lut["lut_out"])
        lut["gram_out"] = ops.linear(w_o_t, w_o_t)
        kvp = t["kv_proj"].to(dev)
        wdt = torch.bfloat16 if kvp.dtype == torch.bfloat16 else torch.float32
        lut["wv_t"] = kvp[kh:].to(wdt).view(self.kv, self.hd, self.dt).transpose(1, 2).contiguous()  # [kv, Dt, hd]
        lut["mem_norm"] = t["mem_norm"].to(dev, torch.float32).contiguous()
        self.wv_dtype = ops.dtype_code(wdt)
        self.luts = lut
        del ef

    @staticmethod
    def _pack_tiles(x: torch.Tensor) -> torch.Tensor:
        """``[V, I]`` fp32 -> ``lng_drafter.lut_out_pk`` order ``[ceil(V/16)][I/16][64][4]`` (a permutation;
        zero rows pad V to a multiple of 16)."""
        v, i = x.shape
        vp = -(-v // 16) * 16
        xp = torch.zeros(vp, i, dtype=x.dtype, device=x.device)
        xp[:v] = x
        # (tile, col, step, kq, e) -> (tile, step, kq, col, e); lane = 16 kq + col
        return xp.view(vp // 16, 16, i // 16, 4, 4).permute(0, 2, 3, 1, 4).contiguous().view(-1)

    def _descriptor(self, tok, codes, ssm, length, rows) -> _lib.Drafter:
        c = self.cfg
        D = _lib.Drafter()
        D.d, D.V, D.R, D.bits, D.mem_dim, D.dt = self.d, self.V, self.R, self.bits, self.mem_dim, self.dt
        D.n_orders = len(self.ngrams)
        for i, n in enumerate(self.ngrams):
            D.orders[i] = n
            D.tables[i] = self.tables[i].data_ptr()
        D.maxn = self.maxn
        D.q_heads, D.kv_heads, D.head_dim, D.ssm_dim = self.qh, self.kv, self.hd, self.N
        D.router_ssm, D.query_ssm = int(self.router_ssm), int(self.query_ssm)
        D.emb_dtype, D.table_dtype, D.router_dtype = _dt(self.emb), _dt(self.tables[0]), _dt(self.router)
        D.router_eps, D.ssm_eps = float(c["router_eps"]), float(c.get("ssm_eps", c["router_eps"]))
        D.draft_eps, D.mem_eps, D.sink_logit = float(c["draft_eps"]), float(c["mem_eps"]), float(c["sink_logit"])
        D.emb, D.router = self.emb.data_ptr(), self.router.data_ptr()
        for k in ("router_start", "router_prev_norm", "router_cur_norm", "out_norm"):
            setattr(D, k, self.vec[k].data_ptr())
        if self.N:
            for k in ("ssm_norm", "ssm_w_in", "ssm_decay"):
                setattr(D, k, self.vec[k].data_ptr())
        D.qk, D.ov = self.qk.data_ptr(), self.ov.data_ptr()
        D.qks = self.qks.data_ptr() if self.qks is not None else None
        D.tokens, D.codes, D.ssm, D.length = tok.data_ptr(), codes.data_ptr(), ssm.data_ptr(), length.data_ptr()
        D.rows = rows
        D.sync = self.sync.data_ptr()
        if self.luts is not None:
            for k, v in self.luts.items():
                setattr(D, k, v.data_ptr())
            D.wv_dtype = self.wv_dtype
        return D

    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    @staticmethod
    def _i32(vals) -> ctypes.Array:
        return (ctypes.c_int32 * max(len(vals), 1))(*[int(v) for v in vals])

    # ------------------------------------------------------------------ state
    def reset(self) -> None:
        with self._lock:
            self._tokens: list = []
            self.len_d.zero_()

    @property
    def length(self) -> int:
        return len(self._tokens)

    @property
    def tokens(self) -> list:
        return list(self._tokens)

    def committed_codes(self) -> np.ndarray:
        return self.codes_d[: self.length].cpu().numpy()

    def truncate(self, length: int) -> None:
        if not 0 <= length <= self.length:
            raise ValueError(f"cannot truncate to {length} (length {self.length})")
        with self._lock:
            del self._tokens[length:]
            self.len_d.fill_(length)

    def _check_tokens(self, toks) -> list:
        toks = [int(x) for x in toks]
        for x in toks:
            if not 0 <= x < self.V:
                raise ValueError(f"token id {x} out of range [0, {self.V})")
        return toks

    def commit(self, tokens, codes=None) -> None:
        """Append verified tokens; ``codes`` [n, R] (optional) replace the drafter's own codes."""
        toks = self._check_tokens(tokens)
        n = len(toks)
        if n == 0:
            return
        with self._lock:
            L = self.length
            if L + n > self.max_len:
                raise ValueError(f"context full: {L} + {n} > {self.max_len}")
            self.tok_d[L:L + n] = torch.tensor(toks, dtype=torch.int64).to(self.device)
            if codes is not None:
                ca = np.asarray(codes)
                if ca.shape != (n, self.R):
                    raise ValueError(f"codes must be [{n}, {self.R}]")
                if (ca < 0).any() or (ca >= 1 << self.bits).any():
                    raise ValueError(f"codes must lie in [0, {1 << self.bits})")
                self.codes_d[L:L + n] = torch.from_numpy(ca.astype(np.uint8)).to(self.device)
            check(self.lib.lng_drafter_advance_range(ctypes.byref(self.D), L, -1 if L > 0 else ROW_NONE, n,
                                                     int(codes is None), self.work.data_ptr(), self.work.numel(),
                                                     self._stream()), "drafter commit")
            self._tokens.extend(toks)
            self.len_d.fill_(L + n)

    # ------------------------------------------------------------------ drafting
    def _window(self, seq: list) -> list:
        w = seq[-self.maxn:]
        return [ROW_NONE] * (self.maxn - len(w)) + w

    def draft(self, gamma: int, hyp=(), topk: int | None = None, last_codes: bool = False) -> DraftOut:
        """``gamma`` greedy drafts after the committed tokens + ``hyp`` (nothing is committed)."""
        k = int(topk or self.topk)
        if not 1 <= k <= _MAX_K:
            raise ValueError(f"topk must be in [1, {_MAX_K}]")
        hyp = self._check_tokens(hyp)
        gamma = int(gamma)
        with self._lock:
            L = self.length
            if L == 0 and not hyp:
                raise ValueError("draft needs at least one committed or hypothetical token")
            nh = len(hyp)
            if nh + gamma + 1 > _HYP_ROWS:
                raise ValueError(f"len(hyp) + gamma must stay below {_HYP_ROWS}")
            lib, Dp, st = self.lib, ctypes.byref(self.D), self._stream()
            wp, wb = self.work.data_ptr(), self.work.numel()
            base = self.hyp_row0
            seq = [-i for i in range(min(L, self.maxn), 0, -1)]  # committed rows relative to L
            if nh:
                self.tok_d[base:base + nh] = torch.tensor(hyp, dtype=torch.int64).to(self.device)
                check(lib.lng_drafter_advance_range(Dp, base, -1 if L > 0 else ROW_NONE, nh, 1, wp, wb, st),
                      "drafter advance")
                seq += [base + j for j in range(nh)]
            advanced = 0
            for i in range(gamma):
                nxt = base + nh + i
                child = i + 1 < gamma or last_codes
                win = self._i32(self._window(seq))
                cr, cp, ck = self._i32([nxt]), self._i32([0]), self._i32([0])
                if self.sketch is None:
                    check(lib.lng_drafter_readout(Dp, win, 1, k, int(self.online), self.kappa, cr, cp, ck, int(child),
                                                  wp, wb, self.counts.data_ptr(), self.ids_d[i].data_ptr(),
                                                  self.sc_d[i].data_ptr(), None, st), "drafter readout")
                else:
                    check(lib.lng_drafter_readout_shortlist(Dp, ctypes.byref(self.sketch), win, 1, k, cr, cp, ck,
                                                            int(child), wp, wb, self.ids_d[i].data_ptr(),
                                                            self.sc_d[i].data_ptr(), None, None, st),
                          "drafter readout + shortlist")
                if child:
                    check(lib.lng_drafter_advance(Dp, self._i32([nxt]), self._i32([seq[-1]]), 1, 1, wp, wb, st),
                          "drafter advance")
                    seq.append(nxt)
                    advanced += 1
            ids, lg, codes = self._fetch(gamma, k, base, nh + advanced)
        if gamma and (ids[:, 0] == -2).any():
            raise RuntimeError("drafter select: candidate buffer overflow (context too long for online counts)")
        lg[ids < 0] = -np.inf
        return DraftOut([int(x) for x in ids[:, 0]], ids, lg.astype(np.float32), codes)

    def _fetch(self, gamma: int, k: int, row0: int, nrows: int):
        """Top-k ids [gamma, k], scores [gamma, k] and the codes of rows row0 .. row0+nrows-1 on the
        host, through one device-to-host copy."""
        n_ids, n_sc, n_c = gamma * k * 8, gamma * k * 4, nrows * self.R
        total = n_ids + n_sc + n_c
        d = self._out_d
        d[:n_ids].view(torch.int64).view(gamma, k).copy_(self.ids_d[:gamma, :k])
        d[n_ids:n_ids + n_sc].view(torch.float32).view(gamma, k).copy_(self.sc_d[:gamma, :k])
        d[n_ids + n_sc:total].view(nrows, self.R).copy_(self.codes_d[row0: row0 + nrows])
        h = self._out_h
        h[:total].copy_(d[:total], non_blocking=True)
        torch.cuda.current_stream(self.device).synchronize()
        a = h[:total].numpy()
        ids = a[:n_ids].view(np.int64).reshape(gamma, k).copy()
        lg = a[n_ids:n_ids + n_sc].view(np.float32).reshape(gamma, k).copy()
        codes = a[n_ids + n_sc:total].reshape(nrows, self.R).copy()
        return ids, lg, codes

    def draft_tree(self, spec) -> list:
        """``draft_tree`` (``drafting/tree.py:243-257``) with every parent of one depth in one readout;
        returns the node tokens (root = the last committed token).  The node tokens and the
        one-launch tree's error word leave the device in one copy; if a wait of the one-launch tree
        ran out, its workspace is cleared and the tree is drafted again by the per-depth readouts."""
        self.tree_step(spec, route_tokens=False)
        rows = slice(self.tree_row0, self.tree_row0 + spec.n)
        if self.level_work is None or not self._level_specs.get((tuple(spec.parent), tuple(spec.rank)), False):
            return self.tok_d[rows].cpu().tolist()
        both = torch.cat((self.tok_d[rows], self.tree_status().to(torch.int64))).cpu().tolist()
        if both[-1] == 0:
            return both[:-1]
        self.level_work.zero_()
        self._redo_per_depth(spec, None)
        return self.tok_d[rows].cpu().tolist()

    def tree_status(self) -> torch.Tensor:
        """The one-launch tree's error word as a device int32 ``[1]`` view (no synchronisation): a
        caller of :meth:`tree_step` copies it to the host with its own results; non-zero means a wait
        of that call ran out and its outputs are not to be used (clear it with :meth:`tree_error` and
        redo the step).  Zero for drafters without the one-launch tree."""
        if self.level_work is None:
            return torch.zeros(1, dtype=torch.int32, device=self.device)
        return self.level_work[4:8].view(torch.int32)

    def tree_step(self, spec, route_tokens: bool = True, graph: bool = False):
        """Draft the tree on the device and (optionally) gather its verification route tokens
        ``[n, R, Dt]``; returns (node tokens int64 [n] (device view), route tokens or None).
        No host synchronisation: the one-launch tree's error word is :meth:`tree_status`.

        ``graph=True`` replays the step's launches from a HIP graph captured on the first call for
        this tree shape (the launches read the drafter state from device memory, so one capture
        serves every later step).  The route tokens then live in a buffer owned by the capture:
        each replay overwrites the previous step's."""
        if graph:
            key = (tuple(spec.parent), tuple(spec.rank), bool(route_tokens))
            ent = self._graphs.get(key)
            if ent is None:
                self.tree_step(spec, route_tokens)          # eager once: argument errors surface here
                torch.cuda.synchronize(self.device)
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    node, out = self.tree_step(spec, route_tokens)
                ent = self._graphs[key] = (g, out)
            ent[0].replay()
            return self.tok_d[self.tree_row0: self.tree_row0 + spec.n], ent[1]
        n = spec.n
        if n > _TREE_ROWS:
            raise ValueError(f"at most {_TREE_ROWS} tree nodes")
        if self.length == 0:
            raise ValueError("draft_tree needs at least one committed token")
        out = None
        if route_tokens:
            out = torch.empty(n, self.R, self.dt, dtype=self.tables[0].dtype, device=self.device)
        parent, rank = self._i32(spec.parent), self._i32(spec.rank)
        key = (tuple(spec.parent), tuple(spec.rank))
        if self.level_work is not None and self._level_specs.get(key, True):
            rc = self.lib.lng_drafter_tree_levels(ctypes.byref(self.D), parent, rank, n, self.tree_row0,
                                                  int(self.online), self.kappa, self.level_work.data_ptr(),
                                                  self.level_work.numel(),
                                                  out.data_ptr() if out is not None else None, self._stream())
            if rc == 0:
                self._level_specs[key] = True
                return self.tok_d[self.tree_row0: self.tree_row0 + n], out
            if rc != _lib.E_ARG:
                check(rc, "drafter tree (one-launch tree, lng_drafter_tree_levels)")
            self._level_specs[key] = False     # tree outside the one-launch kernel's limits
        self._redo_per_depth(spec, out)
        return self.tok_d[self.tree_row0: self.tree_row0 + n], out

    def _redo_per_depth(self, spec, out) -> None:
        """The tree by the per-depth readouts (``lng_drafter_tree``, or its shortlist form)."""
        parent, rank = self._i32(spec.parent), self._i32(spec.rank)
        n = spec.n
        if self.sketch is not None:
            check(self.lib.lng_drafter_tree_shortlist(ctypes.byref(self.D), ctypes.byref(self.sketch), parent, rank, n,
                                                      self.tree_row0, self.work.data_ptr(), self.work.numel(),
                                                      self.sl_lg.data_ptr(),
                                                      out.data_ptr() if out is not None else None, self._stream()),
                  "drafter tree")
            return
        check(self.lib.lng_drafter_tree(ctypes.byref(self.D), parent, rank, n, self.tree_row0, int(self.online),
                                        self.kappa, self.work.data_ptr(), self.work.numel(), self.counts.data_ptr(),
                                        out.data_ptr() if out is not None else None, self._stream()),
              "drafter tree")

    def tree_error(self) -> int:
        """Error word of the one-launch tree (synchronises): 0 = ok; non-zero clears the workspace
        and raises."""
        if self.level_work is not None:
            err = int(self.tree_status().item())
            if err:
                self.level_work.zero_()
                raise RuntimeError(f"drafter tree (one-launch tree, lng_drafter_tree_levels): a device wait ran "
                                   f"out (error word {err})")
        return 0

    def trace(self, tokens, codes=None, full: bool = False):
        """Teacher-forced pass from an empty state: (codes [T, R] uint8, ids [T, S] int64,
        logits [T, S] fp32), S = the vocabulary, or the shortlist cap when the drafter scores a
        sketch shortlist and ``full`` is off (``RefDrafter.trace``, ``cpu_drafter.py:272-289``:
        candidate order, -1 / -inf pad).  The committed state is untouched."""
        toks = self._check_tokens(tokens)
        T = len(toks)
        dev = self.device
        tok = torch.tensor(toks, dtype=torch.int64).to(dev)
        cod = torch.zeros(max(T, 1), self.R, dtype=torch.uint8, device=dev)
        ssm = torch.zeros(max(T, 1), max(self.N, 1), dtype=torch.float32, device=dev)
        ln = torch.zeros(1, dtype=torch.int32, device=dev)
        D = self._descriptor(tok if T else torch.zeros(1, dtype=torch.int64, device=dev), cod, ssm, ln, max(T, 1))
        logits = torch.empty(T, self.V, dtype=torch.float32, device=dev)
        ids = torch.empty(16, 1, dtype=torch.int64, device=dev)
        sc = torch.empty(16, 1, dtype=torch.float32, device=dev)
        short = self.sketch is not None and not full
        if short:
            sl = torch.empty(max(T, 1), self.cap, dtype=torch.int32, device=dev)
            sll = torch.empty(max(T, 1), self.cap, dtype=torch.float32, device=dev)
            ids2 = torch.empty(16, 1, dtype=torch.int64, device=dev)
            sc2 = torch.empty(16, 1, dtype=torch.float32, device=dev)
        nbytes = self.lib.lng_drafter_workspace_bytes(ctypes.byref(D), 16, 1, max(T, 1))
        work = torch.empty(int(nbytes), dtype=torch.uint8, device=dev)
        st = self._stream()
        with self._lock:
            if codes is not None:
                ca = np.asarray(codes)
                if ca.shape != (T, self.R):
                    raise ValueError(f"codes must be [{T}, {self.R}]")
                if (ca < 0).any() or (ca >= 1 << self.bits).any():
                    raise ValueError(f"codes must lie in [0, {1 << self.bits})")
                cod[:T] = torch.from_numpy(ca.astype(np.uint8)).to(dev)
            if T:
                check(self.lib.lng_drafter_advance_range(ctypes.byref(D), 0, ROW_NONE, T, int(codes is None),
                                                         work.data_ptr(), work.numel(), st), "drafter trace")
            chunk = max(1, min(16, 61440 // (4 * max(self.d + self.N, self.qh * self.dt))))
            for t0 in range(0, T, chunk):
                P = min(chunk, T - t0)
                win = []
                for t in range(t0, t0 + P):
                    win += [s if s >= 0 else ROW_NONE for s in range(t - self.maxn + 1, t + 1)]
                check(self.lib.lng_drafter_readout(ctypes.byref(D), self._i32(win), P, 1, 0, 0.0, None, None, None, 0,
                                                   work.data_ptr(), work.numel(), None, ids.data_ptr(), sc.data_ptr(),
                                                   logits[t0].data_ptr(), st), "drafter trace")
                if short:
                    check(self.lib.lng_drafter_shortlist(ctypes.byref(D), ctypes.byref(self.sketch), self._i32(win), P,
                                                         logits[t0].data_ptr(), ids.data_ptr(), sc.data_ptr(), 1, None,
                                                         None, None, 0, ids2.data_ptr(), sc2.data_ptr(),
                                                         sl[t0].data_ptr(), sll[t0].data_ptr(), st), "drafter trace")
            out_c = cod[:T].cpu().numpy()
            if short:
                return out_c, sl[:T].long().cpu().numpy(), sll[:T].cpu().numpy()
            out_l = logits.cpu().numpy()
        out_i = np.broadcast_to(np.arange(self.V, dtype=np.int64), (T, self.V)).copy()
        return out_c, out_i, out_l
