"""ctypes binding of ``liblngram_hip.so`` (the gfx950 C ABI declared in ``include/lngram_hip.h``).

The library is loaded after ``torch`` so that it binds to the HIP runtime torch has
already loaded (same SONAME), which makes torch's stream handles valid arguments.
There is no fallback: if the library is missing, every op raises.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime this library must share)

LIB_PATH = Path(__file__).resolve().parent / "liblngram_hip.so"

# dtype codes (include/lngram_hip.h)
F32, BF16, F16, U8, I32, I64 = 0, 1, 2, 3, 4, 5

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f = ctypes.c_float
_int = ctypes.c_int
_P64 = ctypes.POINTER(ctypes.c_int64)
_P32 = ctypes.POINTER(ctypes.c_int32)

E_ARG = -1  # LNG_E_ARG
ROW_NONE = -2147483648  # LNG_ROW_NONE
NORM_MODEL, NORM_FUSED = 0, 1  # LNG_NORM_MODEL / LNG_NORM_FUSED
DR_SYNC_INTS = 4160  # LNG_DR_SYNC_INTS
READOUT_PACK_ELEMS = 131072  # LNG_READOUT_PACK_ELEMS: bf16 elements of the fused readout's packed KV weight


class Drafter(ctypes.Structure):
    """``lng_drafter`` (include/lngram_hip.h): shapes, device weight pointers and state rows."""

    _fields_ = [(n, ctypes.c_int32) for n in ("d", "V", "R", "bits", "mem_dim", "dt", "n_orders")] + [
        ("orders", ctypes.c_int32 * 4), ("maxn", ctypes.c_int32)] + [
        (n, ctypes.c_int32) for n in ("q_heads", "kv_heads", "head_dim", "ssm_dim", "router_ssm", "query_ssm",
                                      "emb_dtype", "table_dtype", "router_dtype")] + [
        (n, ctypes.c_float) for n in ("router_eps", "ssm_eps", "draft_eps", "mem_eps", "sink_logit")] + [
        ("emb", ctypes.c_void_p), ("tables", ctypes.c_void_p * 4), ("router", ctypes.c_void_p)] + [
        (n, ctypes.c_void_p) for n in ("router_start", "router_prev_norm", "router_cur_norm", "ssm_norm", "ssm_w_in",
                                       "ssm_decay", "qk", "qks", "ov", "out_norm", "tokens", "codes", "ssm",
                                       "length")] + [("rows", ctypes.c_int32)] + [
        (n, ctypes.c_void_p) for n in ("lut_prev", "lut_cur", "lut_start", "lut_qk", "lut_out", "gram_out", "wv_t",
                                       "mem_norm")] + [("wv_dtype", ctypes.c_int32), ("sync", ctypes.c_void_p),
                                                        ("lut_out_pk", ctypes.c_void_p)]


_PD = ctypes.POINTER(Drafter)


class Sketch(ctypes.Structure):
    """``lng_sketch`` (include/lngram_hip.h): device count sketches of the drafter's orders."""

    _fields_ = [("ids", ctypes.c_void_p * 4), ("counts", ctypes.c_void_p * 4), ("k", ctypes.c_int32),
                ("cap", ctypes.c_int32), ("fallback", ctypes.c_void_p), ("n_fallback", ctypes.c_int32)]


_PS = ctypes.POINTER(Sketch)

# name -> (restype, argtypes); must cover every function declared in the header
SIGNATURES = {
    "lng_abi_version": (_int, []),
    "lng_last_error": (ctypes.c_char_p, []),
    "lng_router_codes": (_int, [_p, _int, _p, _int, _i64, _i64, _i64, _i32, _p, _p, _int, _p]),
    "lng_pack_route_codes": (_int, [_p, _i64, _i64, _i32, _p, _int, _p]),
    "lng_router_features": (_int, [_p, _int, _p, _i64, _i64, _i64, _i32, _p, _p, _p, _f, _p, _i32, _p, _p]),
    "lng_router_feature_tables": (_int, [_p, _i64, _i32, _p, _p, _p, _f, _p, _p, _p]),
    "lng_router_codes_ids_ok": (_i32, [_i64, _i32, _i32, _i64]),
    "lng_router_codes_ids": (_int, [_p, _i64, _i64, _i64, _p, _p, _i32, _p, _i32, _p, _i64, _p, _p, _p]),
    "lng_ngram_address": (_int, [_p, _int, _i64, _i64, _i32, _i32, _i32, _p, _int, _p]),
    "lng_ngram_rows": (_int, [_p, _int, _i64, _i64, _i32, _i32, _i32, _P32, _i32, _i32, _p, _p, _p, _int, _p]),
    "lng_online_mix": (_int, [_p, _p, _i32, _p, _p, _i32, _i32, _i32, _p, _i64, _f, _p, _p, _p]),
    "lng_route_tokens": (_int, [_p, _int, _i64, _i64, _i32, _i32, _i32, _P32, _i32, _i32,
                                ctypes.POINTER(_p), _int, _i32, _p, _p, _i32, _p, _p]),
    "lng_rmsnorm": (_int, [_p, _p, _int, _i64, _i32, _f, _i32, _p, _p]),
    "lng_linear": (_int, [_p, _p, _int, _i64, _i64, _i64, _p, _p]),
    "lng_linear_at": (_int, [_p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _p]),
    "lng_router_codes_at": (_int, [_p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _p]),
    "lng_sink_attention": (_int, [_p, _p, _p, _int, _i64, _i32, _i32, _i32, _i32, _f, _f, _p, _p]),
    "lng_sink_attention_strided": (_int, [_p, _p, _p, _int, _i64, _i32, _i32, _i32, _i32, _P64, _P64,
                                          _f, _f, _p, _p]),
    "lng_sink_probabilities": (_int, [_p, _i64, _i32, _f, _p, _p]),
    "lng_causal_conv": (_int, [_p, _p, _p, _int, _i64, _i64, _i32, _i32, _i32, _f, _int, _p, _p]),
    "lng_causal_conv_at": (_int, [_p, _p, _p, _int, _i64, _i64, _i64, _i64, _p, _i64, _i32, _i32, _i32, _f, _int, _p,
                                  _p]),
    "lng_causal_conv_slots": (_int, [_p, _p, _p, _int, _i64, _i64, _i64, _p, _i64, _i32, _i32, _i32, _i32, _f, _int,
                                      _p, _p]),
    "lng_linear_rowsq_partials": (_i32, [_i64]),
    "lng_linear_rowsq": (_int, [_p, _p, _i64, _i64, _i64, _p, _p, _p]),
    "lng_linear_rowscale_ok": (_i32, [_i64, _i64, _i64]),
    "lng_linear_rowscale": (_int, [_p, _p, _i64, _i64, _i64, _f, _p, _p]),
    "lng_row_sumsq": (_int, [_p, _i64, _i32, _p, _p]),
    "lng_causal_conv_rowsq": (_int, [_p, _p, _i32, _p, _p, _i64, _i64, _i32, _i32, _i32, _f, _int, _p, _p]),
    "lng_memory_readout_fused": (_int, [_p, _p, _f, _p, _i64, _i64, _i32, _p, _p, _p, _p, _f, _f, _f, _p, _p]),
    "lng_memory_readout_fused_at": (_int, [_p, _p, _f, _p, _i64, _i64, _i32, _i64, _i64, _p, _p, _p, _p, _p, _f, _f,
                                           _f, _p, _p]),
    "lng_memory_readout_fused_rows": (_int, [_p, _p, _f, _p, _i64, _i64, _i32, _p, _p, _f, _f, _f, _p, _p]),
    "lng_fold_columns": (_int, [_p, _p, _i64, _i64, _p, _p]),
    "lng_memory_readout_pack": (_int, [_p, _p, _p]),
    "lng_gather_sum_scaled": (_int, [ctypes.POINTER(_p), _int, _i32, _p, _i64, _i64, _i32, _P32, _i32, _i32, _i32,
                                     ctypes.c_uint32, _p, _p]),
    "lng_surrogate_grad": (_int, [_p, _p, _int, _p, _int, _p, _int, _p, _i64, _p, _i64, _i64, _i32, _i32, _i32,
                                  _i32, _i32, _f, _f, _int, _p, _int, _p]),
    "lng_tree_windows": (_int, [_p, _int, _p, _i64, _i64, _i32, _i32, _i32, _p, _i64, _p, _p, _i32, _p, _p, _p, _p,
                                _p]),
    "lng_surrogate_workspace_bytes": (ctypes.c_size_t, [_i64, _i64, _i32, _i32, _i32, _i32, _int, _int]),
    "lng_surrogate_grad_ws": (_int, [_p, _p, _int, _p, _int, _p, _int, _p, _i64, _p, _i64, _i64, _i32, _i32, _i32, _i32,
                                     _i32, _f, _f, _int, _p, ctypes.c_size_t, _p, _int, _p]),
    "lng_table_grad": (_int, [_p, _int, _p, _int, _p, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _i64, _p, _p]),
    "lng_host_device_pointer": (_int, [_p, ctypes.POINTER(_p)]),
    "lng_permute_table": (_int, [_p, _p, _int, _i32, _i32, _i32, _i32, _p]),
    "lng_serving_address": (_int, [_p, _int, _i64, _i64, _i32, _i32, _i32, _p, _p]),
    "lng_serving_gather": (_int, [ctypes.POINTER(_p), _P64, _int, _i32, _P32, _i32, _i32, _p, _int, _i64, _i64, _i64,
                                  _i32, _i64, _p, _p]),
    "lng_serving_candidates": (_int, [ctypes.POINTER(_p), _P64, _int, _i32, _P32, _i32, _i32, _p, _int, _i64, _i64,
                                      _i32, _i64, _p, _p]),
    "lng_gather_rows": (_int, [_p, _i64, _int, _i32, _p, _i64, _p, _p]),
    "lng_select_candidates": (_int, [_p, _int, _i32, _p, _int, _i64, _i32, _i32, _i32, _p, _p]),
    "lng_ssm_workspace_bytes": (ctypes.c_size_t, [_i64, _i64, _i32]),
    "lng_ssm_scan": (_int, [_p, _p, _p, _i64, _i64, _i32, _p, ctypes.c_size_t, _p, _p]),
    "lng_ssm_scan_bounded": (_int, [_p, _p, _p, _i64, _i64, _i32, _p, ctypes.c_size_t, _i32, _p, _p]),
    "lng_ssm_scan_with_bf16": (_int, [_p, _p, _p, _i64, _i64, _i32, _p, ctypes.c_size_t, _p, _p, _p]),
    "lng_ssm_tree": (_int, [_p, _p, _p, _p, _i64, _i32, _i32, _p, _p]),
    "lng_ssm_scan_static": (_int, [_p, _p, _p, _i64, _i64, _i32, _p, _p]),
    "lng_ssm_scan_static_status": (_int, [_p]),
    "lng_drafter_tree_levels_workspace": (ctypes.c_size_t, [_PD]),
    "lng_drafter_tree_levels": (_int, [_PD, _P32, _P32, _i32, _i32, _int, _f, _p, ctypes.c_size_t, _p, _p]),
    "lng_tree_accept": (_int, [_p, _p, _p, _i32, _p, _p, _p, _p]),
    "lng_drafter_size": (ctypes.c_size_t, []),
    "lng_drafter_workspace_bytes": (ctypes.c_size_t, [_PD, _i32, _i32, _i32]),
    "lng_drafter_advance": (_int, [_PD, _P32, _P32, _i32, _int, _p, ctypes.c_size_t, _p]),
    "lng_drafter_advance_range": (_int, [_PD, _i32, _i32, _i32, _int, _p, ctypes.c_size_t, _p]),
    "lng_drafter_readout": (_int, [_PD, _P32, _i32, _i32, _int, _f, _P32, _P32, _P32, _i32, _p, ctypes.c_size_t,
                                   _p, _p, _p, _p, _p]),
    "lng_drafter_gather": (_int, [_PD, _P32, _i32, _p, _p]),
    "lng_drafter_shortlist": (_int, [_PD, _PS, _P32, _i32, _p, _p, _p, _i32, _P32, _P32, _P32, _i32, _p, _p, _p, _p,
                                     _p]),
    "lng_drafter_readout_shortlist": (_int, [_PD, _PS, _P32, _i32, _i32, _P32, _P32, _P32, _i32, _p, ctypes.c_size_t,
                                             _p, _p, _p, _p, _p]),
    "lng_drafter_tree": (_int, [_PD, _P32, _P32, _i32, _i32, _int, _f, _p, ctypes.c_size_t, _p, _p, _p]),
    "lng_drafter_tree_shortlist": (_int, [_PD, _PS, _P32, _P32, _i32, _i32, _p, ctypes.c_size_t, _p, _p, _p]),
}

_lock = threading.Lock()
_lib = None


class LibraryMissing(RuntimeError):
    pass


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """The loaded library (loaded once).  Raises ``LibraryMissing`` if it was not built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        p = Path(path) if path else LIB_PATH
        if not p.exists():
            raise LibraryMissing(f"{p} not built: run `python lngram-decode_amd/build.py` "
                                 "(or __graft_entry__.build()); there is no CPU fallback")
        lib = ctypes.CDLL(str(p))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().lng_last_error()
        raise RuntimeError(f"{what} failed ({rc}): {msg.decode() if msg else ''}")
