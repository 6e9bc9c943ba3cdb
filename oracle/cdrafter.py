"""ctypes loader of the oracle's C++ CPU drafter port (``oracle/c/cpu_drafter.cpp``) -- test
infrastructure only: the drafter CPU baseline of ``bench.py`` and a second restatement of the
draft head that the tests compare with ``oracle.drafting.DrafterOracle``.

``CppDrafterPort(config, tensors, threads, online, kappa)`` takes a drafter bundle (the
``(config, tensors)`` pair of ``drafting/export_drafter.py``) and mirrors the reference drafter API
(``drafting/cpu_drafter.py:76-289``): ``reset / length / tokens / truncate / commit / draft /
trace`` plus ``draft_tree`` (``drafting/tree.py:243-257``).
"""

from __future__ import annotations

import ctypes
import os

import numpy as np
import torch

from . import cint
from .drafting import DraftOut

LIB = cint.HERE / "_build" / "libcpu_drafter.so"
_lib = None


class _Config(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("d", "V", "R", "bits", "mem_dim", "kv_heads", "head_dim", "q_heads",
                                               "ssm_dim", "n_orders")] + [("orders", ctypes.c_int32 * 4)] + [
        (n, ctypes.c_int32) for n in ("router_ssm", "query_ssm", "table_bf16")] + [
        (n, ctypes.c_float) for n in ("router_eps", "ssm_eps", "draft_eps", "mem_eps", "softmax_scale", "sink_logit")]


_WEIGHTS = ("embedding", "mem_norm", "kv_proj", "router", "router_prev_norm", "router_cur_norm", "router_start",
            "ssm_norm", "ssm_w_in", "ssm_decay", "q_norm", "w_q", "w_sq", "w_o", "out_norm")


class _Weights(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in _WEIGHTS] + [("tables", ctypes.c_void_p * 4)]


def load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            cint.build()
        lib = ctypes.CDLL(str(LIB))
        P, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
        sig = {
            "cdr_last_error": (ctypes.c_char_p, []),
            "cdr_create": (P, [ctypes.POINTER(_Config), ctypes.POINTER(_Weights), ctypes.c_int, ctypes.c_int,
                               ctypes.c_float]),
            "cdr_destroy": (None, [P]),
            "cdr_length": (i64, [P]),
            "cdr_set_threads": (None, [P, ctypes.c_int]),
            "cdr_reset": (None, [P]),
            "cdr_truncate": (ctypes.c_int, [P, i64, i32, i32]),
            "cdr_commit": (ctypes.c_int, [P, P, i64, P]),
            "cdr_draft": (ctypes.c_int, [P, ctypes.c_int, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P, P, P,
                                         ctypes.POINTER(ctypes.c_int)]),
            "cdr_trace": (ctypes.c_int, [P, P, i64, P, P, P]),
            "cdr_draft_tree": (ctypes.c_int, [P, P, P, ctypes.c_int, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


class CppDrafterPort:
    """The drafter API over the C++ port; ``threads`` OpenMP threads (routes and vocabulary)."""

    name = "cpp_port"

    def __init__(self, config: dict, tensors: dict, threads: int | None = None, online: bool = False,
                 kappa: float = 1.0, topk: int = 3):
        c = dict(config)
        self.cfg = c
        self.topk = int(topk)
        self.threads = int(threads or len(os.sched_getaffinity(0)))
        ngrams = [int(n) for n in c["ngrams"]]
        self.R, self.V = int(c["routes"]), int(c["vocab"])
        self.N = int(c.get("ssm_dim", 0) or 0) if "ssm_w_in" in tensors else 0
        tdt = tensors[f"table_{ngrams[0]}"].dtype
        cfg = _Config(d=int(c["d_model"]), V=self.V, R=self.R, bits=int(c["bits"]), mem_dim=int(c["mem_dim"]),
                      kv_heads=int(c["kv_heads"]), head_dim=int(c["head_dim"]), q_heads=int(c["q_heads"]),
                      ssm_dim=self.N, n_orders=len(ngrams), router_ssm=int(c["router_kind"] == "embed2_ssm"),
                      query_ssm=int("w_sq" in tensors), table_bf16=int(tdt == torch.bfloat16),
                      router_eps=float(c["router_eps"]), ssm_eps=float(c.get("ssm_eps", c["router_eps"])),
                      draft_eps=float(c["draft_eps"]), mem_eps=float(c["mem_eps"]),
                      softmax_scale=float(c["softmax_scale"]), sink_logit=float(c["sink_logit"]))
        for i, n in enumerate(ngrams):
            cfg.orders[i] = n
        self._keep = {}
        w = _Weights()
        for k in _WEIGHTS:
            if k in tensors:
                a = np.ascontiguousarray(tensors[k].detach().float().cpu().numpy(), np.float32)
                self._keep[k] = a
                setattr(w, k, a.ctypes.data)
        for i, n in enumerate(ngrams):
            tb = tensors[f"table_{n}"].detach().cpu().contiguous()
            a = tb.view(torch.int16).numpy().view(np.uint16) if tdt == torch.bfloat16 else \
                np.ascontiguousarray(tb.float().numpy(), np.float32)
            self._keep[f"table_{n}"] = a
            w.tables[i] = a.ctypes.data
        self._cfg, self._w = cfg, w
        lib = load()
        self._h = lib.cdr_create(ctypes.byref(cfg), ctypes.byref(w), self.threads, int(online), float(kappa))
        if not self._h:
            raise ValueError(lib.cdr_last_error().decode())
        self._tokens: list = []

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            load().cdr_destroy(h)
            self._h = None

    def _check(self, rc: int) -> None:
        if rc != 0:
            raise RuntimeError(load().cdr_last_error().decode())

    def reset(self) -> None:
        load().cdr_reset(self._h)
        self._tokens = []

    def set_threads(self, threads: int) -> None:
        """OpenMP threads for the later calls."""
        self.threads = max(1, int(threads))
        load().cdr_set_threads(self._h, self.threads)

    @property
    def length(self) -> int:
        return int(load().cdr_length(self._h))

    @property
    def tokens(self) -> list:
        return list(self._tokens)

    def truncate(self, n: int) -> None:
        if not 0 <= n <= self.length:
            raise ValueError(f"cannot truncate to {n} (length {self.length})")
        self._check(load().cdr_truncate(self._h, n, self.R, self.N))
        del self._tokens[n:]

    def commit(self, tokens, codes=None) -> None:
        t = np.ascontiguousarray(np.asarray(tokens, np.int64).reshape(-1))
        c = None if codes is None else np.ascontiguousarray(np.asarray(codes, np.uint8).reshape(len(t), self.R))
        self._check(load().cdr_commit(self._h, _ptr(t), len(t), _ptr(c)))
        self._tokens.extend(int(x) for x in t)

    def draft(self, gamma: int, hyp=(), topk: int | None = None, last_codes: bool = False) -> DraftOut:
        k = int(topk or self.topk)
        hy = np.ascontiguousarray(np.asarray(list(hyp), np.int64))
        toks = np.zeros(max(gamma, 1), np.int64)
        ids = np.full((max(gamma, 1), k), -1, np.int64)
        sc = np.full((max(gamma, 1), k), -np.inf, np.float32)
        codes = np.zeros((len(hy) + gamma + 1, self.R), np.uint8)
        nc = ctypes.c_int(0)
        self._check(load().cdr_draft(self._h, int(gamma), _ptr(hy) if len(hy) else None, len(hy), k, int(last_codes),
                                     _ptr(toks), _ptr(ids), _ptr(sc), _ptr(codes), ctypes.byref(nc)))
        return DraftOut([int(x) for x in toks[:gamma]], ids[:gamma], sc[:gamma], codes[:nc.value])

    def trace(self, tokens, codes=None):
        """(codes [T, R] uint8, scores [T, V] fp32) from an empty state (committed state kept)."""
        t = np.ascontiguousarray(np.asarray(tokens, np.int64).reshape(-1))
        c = None if codes is None else np.ascontiguousarray(np.asarray(codes, np.uint8).reshape(len(t), self.R))
        oc = np.zeros((len(t), self.R), np.uint8)
        ol = np.zeros((len(t), self.V), np.float32)
        self._check(load().cdr_trace(self._h, _ptr(t), len(t), _ptr(c), _ptr(oc), _ptr(ol)))
        return oc, ol

    def draft_tree(self, spec) -> list:
        parent = np.ascontiguousarray(np.asarray(spec.parent, np.int32))
        rank = np.ascontiguousarray(np.asarray(spec.rank, np.int32))
        out = np.zeros(len(parent), np.int64)
        self._check(load().cdr_draft_tree(self._h, _ptr(parent), _ptr(rank), len(parent), _ptr(out)))
        return [int(x) for x in out]
