"""ctypes loader of the oracle's C restatement (``oracle/c/oracle_int.c``) -- test infrastructure only."""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "liboracle_int.so"
_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        _lib = ctypes.CDLL(str(LIB))
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def pack_codes(logits: np.ndarray, bits: int) -> np.ndarray:
    lg = np.ascontiguousarray(logits, np.float32)
    c = lg.shape[-1]
    m = lg.size // c
    out = np.zeros(lg.shape[:-1] + (c // bits,), np.int32)
    load().orc_pack_codes(_p(lg), ctypes.c_int64(m), ctypes.c_int32(c // bits), ctypes.c_int32(bits), _p(out))
    return out


def ngram_rows(codes: np.ndarray, orders, bits: int, segment_ids=None, valid_tokens=None) -> np.ndarray:
    c = np.ascontiguousarray(codes, np.int32)
    b, t, r = c.shape
    ords = np.asarray(orders, np.int32)
    seg = None if segment_ids is None else np.ascontiguousarray(segment_ids, np.int32)
    val = None if valid_tokens is None else np.ascontiguousarray(valid_tokens, np.uint8)
    out = np.zeros((b, t, r, len(ords)), np.int64)
    load().orc_ngram_rows(_p(c), ctypes.c_int64(b), ctypes.c_int64(t), ctypes.c_int32(r), _p(ords),
                          ctypes.c_int32(len(ords)), ctypes.c_int32(bits), None if seg is None else _p(seg),
                          None if val is None else _p(val), _p(out))
    return out


def tree_slots(parent, L: int, back: int):
    p = np.asarray(parent, np.int32)
    n = len(p)
    idx = np.zeros((n, back + 1), np.int64)
    ok = np.zeros((n, back + 1), np.uint8)
    load().orc_tree_slots(_p(p), ctypes.c_int32(n), ctypes.c_int64(L), ctypes.c_int32(back), _p(idx), _p(ok))
    return idx, ok.astype(bool)


def tree_accept(parent, node_tokens, argmax):
    p = np.asarray(parent, np.int32)
    nt = np.asarray(node_tokens, np.int64)
    am = np.asarray(argmax, np.int64)
    n = len(p)
    path = np.zeros(n, np.int32)
    new = np.zeros(n, np.int64)
    lib = load()
    lib.orc_tree_accept.restype = ctypes.c_int32
    ln = lib.orc_tree_accept(_p(p), ctypes.c_int32(n), _p(nt), _p(am), _p(path), _p(new))
    return path[:ln].tolist(), new[:ln].tolist()


def online_weights(keys: np.ndarray, q: np.ndarray, deadline: np.ndarray) -> np.ndarray:
    """keys ``[n_orders, P, R]``, q ``[n_orders, J, R]`` (int64, -1 invalid), deadline ``[J]`` -> w ``[J, P]``."""
    k = np.ascontiguousarray(keys, np.int64)
    qq = np.ascontiguousarray(q, np.int64)
    dl = np.ascontiguousarray(deadline, np.int64)
    no, p, r = k.shape
    j = qq.shape[1]
    w = np.zeros((j, p), np.float32)
    load().orc_online_weights(_p(k), _p(qq), ctypes.c_int32(no), ctypes.c_int64(p), ctypes.c_int64(j),
                              ctypes.c_int32(r), _p(dl), _p(w))
    return w
