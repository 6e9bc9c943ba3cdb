"""Tensor-level wrappers of the gfx950 kernels.

Every op takes device tensors (torch on ROCm), allocates its outputs with torch,
and enqueues the kernel on the current stream of the tensors' device.  CPU tensors
are rejected: there is no CPU path in the product.
"""

from __future__ import annotations

import ctypes
import math
import threading

import torch

from . import _lib
from ._lib import BF16, F16, F32, I32, I64, U8, check

_DT = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16, torch.uint8: U8, torch.int32: I32,
       torch.int64: I64}


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DT[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}") from None


def _dev(*ts) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError("lngram_hip ops need tensors on a ROCm GPU device; there is no CPU path "
                               f"(got a tensor on {t.device})")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} vs {t.device}")
    return dev


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _c(t: torch.Tensor | None) -> torch.Tensor | None:
    """Contiguous with a 16-byte aligned base (vector loads)."""
    if t is None:
        return None
    if not t.is_contiguous() or t.data_ptr() % 16:
        t = t.contiguous()
        if t.data_ptr() % 16:
            t = t.clone()
    return t


def _ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def lib():
    return _lib.load()


class KernelTimer:
    """Records HIP events around the launches of the named ops on their stream while active:
    every launch, or every ``every``-th one (a timing event pair costs a few microseconds of
    device time, so a long timed loop brackets a sample of its launches).

        with ops.KernelTimer("memory_readout_fused", every=5) as kt:
            ...                       # launches 0, 5, 10, ... are bracketed by events
        kt.mean_ms()                  # average device duration per bracketed launch (synchronises)
    """

    _active: list = []

    def __init__(self, *names: str, every: int = 1):
        if every < 1:
            raise ValueError("every must be >= 1")
        self.names = set(names)
        self.every = int(every)
        self.launches = 0
        self.events: list = []

    def __enter__(self):
        KernelTimer._active.append(self)
        return self

    def __exit__(self, *exc):
        KernelTimer._active.remove(self)
        return False

    def durations_ms(self) -> list:
        if self.events:
            self.events[-1][1].synchronize()
        return [s.elapsed_time(e) for s, e in self.events]

    def mean_ms(self) -> float:
        d = self.durations_ms()
        return sum(d) / len(d) if d else float("nan")


def _timed(name: str, dev: torch.device, launch):
    timers = []
    for t in KernelTimer._active:
        if name in t.names:
            if t.launches % t.every == 0:
                timers.append(t)
            t.launches += 1
    if not timers:
        return launch()
    st = torch.cuda.current_stream(dev)
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record(st)
    rc = launch()
    e.record(st)
    for t in timers:
        t.events.append((s, e))
    return rc


# ----------------------------------------------------------------------------- K1
def router_codes(x: torch.Tensor, w: torch.Tensor, bits: int, want_logits: bool = True,
                 codes_dtype: torch.dtype = torch.int32):
    """``(logits fp32 [..., N] or None, codes [..., N/bits])`` for ``x [..., K] . w[N, K]^T``."""
    dev = _dev(x, w)
    x2 = _c(x.reshape(-1, x.shape[-1]))
    w = _c(w)
    m, k = x2.shape
    n = w.shape[0]
    if w.shape[1] != k:
        raise ValueError(f"router weight {tuple(w.shape)} does not match input dim {k}")
    lead = x.shape[:-1]
    logits = torch.empty(*lead, n, dtype=torch.float32, device=dev) if want_logits or not (
        x.dtype == w.dtype == torch.bfloat16 and bits == 4 and k % 8 == 0) else None
    codes = torch.empty(*lead, n // bits, dtype=codes_dtype, device=dev)
    check(lib().lng_router_codes(_ptr(x2), dtype_code(x2.dtype), _ptr(w), dtype_code(w.dtype), m, k, n, bits,
                                 _ptr(logits), _ptr(codes), dtype_code(codes_dtype), _stream(dev)), "router_codes")
    return (logits if want_logits else None), codes


def pack_route_codes(logits: torch.Tensor, bits: int, codes_dtype: torch.dtype = torch.int32) -> torch.Tensor:
    dev = _dev(logits)
    lg = _c(logits.float())
    c = lg.shape[-1]
    if c % bits:
        raise ValueError(f"route logits dim={c} must be divisible by bits={bits}")
    out = torch.empty(*lg.shape[:-1], c // bits, dtype=codes_dtype, device=dev)
    check(lib().lng_pack_route_codes(_ptr(lg), lg.numel() // c, c, bits, _ptr(out), dtype_code(codes_dtype),
                                     _stream(dev)), "pack_route_codes")
    return out


def router_features(emb: torch.Tensor, start: torch.Tensor, prev_w: torch.Tensor, cur_w: torch.Tensor, eps: float,
                    ssm_state: torch.Tensor | None = None, token_ids: torch.Tensor | None = None) -> torch.Tensor:
    """``concat(RMSNorm(E[x_{t-1}] or start), RMSNorm(E[x_t])[, s_t])`` ``[B, T, 2d (+N)]`` in the
    embedding dtype.  ``token_ids [B, T]`` given: ``emb`` is the ``[V, d]`` table (gather fused in);
    otherwise ``emb [B, T, d]`` holds the gathered rows."""
    dev = _dev(emb, start, prev_w, cur_w, ssm_state, token_ids)
    dt = emb.dtype
    d = emb.shape[-1]
    if token_ids is not None:
        b, t = token_ids.shape
        ids = _c(token_ids.to(torch.int64))
        vocab = emb.shape[0]
    else:
        b, t = emb.shape[:2]
        ids, vocab = None, 0
    n = 0
    sc = None
    if ssm_state is not None:
        if ssm_state.shape[:2] != (b, t):
            raise ValueError(f"ssm_state {tuple(ssm_state.shape)} does not match [B, T] = [{b}, {t}]")
        n = ssm_state.shape[-1]
        sc = _c(ssm_state.float())
    ec = _c(emb)
    out = torch.empty(b, t, 2 * d + n, dtype=dt, device=dev)
    check(lib().lng_router_features(_ptr(ec), dtype_code(dt), _ptr(ids), vocab, b, t, d, _ptr(_c(start.to(dt))),
                                    _ptr(_c(prev_w.to(dt))), _ptr(_c(cur_w.to(dt))), eps, _ptr(sc), n, _ptr(out),
                                    _stream(dev)), "router_features")
    return out


def router_feature_tables(emb: torch.Tensor, start: torch.Tensor, prev_w: torch.Tensor, cur_w: torch.Tensor,
                          eps: float) -> tuple:
    """``(fprev [V+2, d], fcur [V+1, d])`` bf16 (``lng_router_feature_tables``): the normalised
    embedding rows of the token router, ``fprev[V]`` the normalised ``start``, the last row of
    each a zero row."""
    dev = _dev(emb, start, prev_w, cur_w)
    if emb.dtype != torch.bfloat16 or emb.dim() != 2:
        raise ValueError("router_feature_tables takes a bf16 [V, d] embedding table")
    v, d = emb.shape
    fprev = torch.empty(v + 2, d, dtype=torch.bfloat16, device=dev)
    fcur = torch.empty(v + 1, d, dtype=torch.bfloat16, device=dev)
    bf = torch.bfloat16
    check(lib().lng_router_feature_tables(_ptr(_c(emb)), v, d, _ptr(_c(start.to(bf))), _ptr(_c(prev_w.to(bf))),
                                          _ptr(_c(cur_w.to(bf))), eps, _ptr(fprev), _ptr(fcur), _stream(dev)),
          "router_feature_tables")
    return fprev, fcur


def router_codes_ids_ok(m: int, d: int, n: int, n_out: int) -> bool:
    """Shapes ``lng_router_codes_ids`` takes (``m`` tokens, ``d``-wide embeddings, ``n`` SSM columns)."""
    return bool(lib().lng_router_codes_ids_ok(m, d, n, n_out))


def router_codes_ids(token_ids: torch.Tensor, fprev: torch.Tensor, fcur: torch.Tensor, ssm_bf16: torch.Tensor | None,
                     w: torch.Tensor, want_logits: bool = False):
    """``(fp32 logits or None, uint8 codes [B, T, n_out/4])`` of the token router over the features
    gathered from the tables inside the GEMM (``lng_router_codes_ids``): equal to
    ``router_codes(router_features(...), w, 4)``."""
    dev = _dev(token_ids, fprev, fcur, ssm_bf16, w)
    b, t = token_ids.shape
    v = fcur.shape[0] - 1
    d = fcur.shape[1]
    n = 0 if ssm_bf16 is None else ssm_bf16.shape[-1]
    if w.dtype != torch.bfloat16 or w.shape[1] != 2 * d + n:
        raise ValueError(f"router weight {tuple(w.shape)} does not take [2d + N] = [{2 * d + n}] bf16 features")
    if ssm_bf16 is not None and (ssm_bf16.dtype != torch.bfloat16 or tuple(ssm_bf16.shape[:2]) != (b, t)):
        raise ValueError("ssm_bf16 must be bf16 [B, T, N]")
    n_out = w.shape[0]
    ids = _c(token_ids.to(torch.int64))
    codes = torch.empty(b, t, n_out // 4, dtype=torch.uint8, device=dev)
    logits = torch.empty(b, t, n_out, dtype=torch.float32, device=dev) if want_logits else None
    check(lib().lng_router_codes_ids(_ptr(ids), v, b, t, _ptr(_c(fprev)), _ptr(_c(fcur)), d,
                                     _ptr(None if ssm_bf16 is None else _c(ssm_bf16)), n, _ptr(_c(w)), n_out,
                                     _ptr(logits), _ptr(codes), _stream(dev)), "router_codes_ids")
    return logits, codes


def router_features_ok(d: int, n: int, dtype: torch.dtype) -> bool:
    """Shapes ``lng_router_features`` takes."""
    es = torch.finfo(dtype).bits // 8 if dtype.is_floating_point else 0
    return dtype in (torch.bfloat16, torch.float32) and (d * es) % 16 == 0 and d * es <= 8192 and \
        ((2 * d + n) * es) % 16 == 0


# ----------------------------------------------------------------------------- K2
def _codes_ok(codes: torch.Tensor) -> torch.Tensor:
    if codes.dtype not in (torch.uint8, torch.int32, torch.int64):
        codes = codes.to(torch.int32)
    return _c(codes)


def ngram_address(codes: torch.Tensor, order: int, bits: int, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    dev = _dev(codes)
    b, t, r = codes.shape
    out_dtype = out_dtype or (torch.int64 if codes.dtype == torch.int64 else torch.int32)
    cc = _codes_ok(codes)
    out = torch.empty(b, max(t - order + 1, 0), r, dtype=out_dtype, device=dev)
    check(lib().lng_ngram_address(_ptr(cc), dtype_code(cc.dtype), b, t, r, order, bits, _ptr(out),
                                  dtype_code(out_dtype), _stream(dev)), "ngram_address")
    return out


def _orders(orders) -> ctypes.Array:
    arr = (ctypes.c_int32 * len(orders))(*[int(o) for o in orders])
    return arr


def _seg(segment_ids, valid_tokens):
    seg = None if segment_ids is None else _c(segment_ids.to(torch.int32))
    val = None if valid_tokens is None else _c(valid_tokens.to(torch.uint8))
    return seg, val


def ngram_rows(codes: torch.Tensor, orders, bits: int, route_start: int = 0, route_end: int | None = None,
               segment_ids=None, valid_tokens=None, rows_dtype: torch.dtype | None = None) -> torch.Tensor:
    """``[B, T, route_end-route_start, len(orders)]`` global rows, -1 where the row is masked.
    int32 unless the largest row needs int64 (the reference's ``index_dtype``,
    ``lngram_v2.py:951-959``) or ``rows_dtype`` asks for int64."""
    dev = _dev(codes, segment_ids, valid_tokens)
    b, t, r = codes.shape
    route_end = r if route_end is None else route_end
    if rows_dtype is None:
        wide = any(r * (1 << (bits * int(n))) - 1 > 2 ** 31 - 1 for n in orders)
        rows_dtype = torch.int64 if wide else torch.int32
    cc = _codes_ok(codes)
    seg, val = _seg(segment_ids, valid_tokens)
    out = torch.empty(b, t, route_end - route_start, len(orders), dtype=rows_dtype, device=dev)
    check(lib().lng_ngram_rows(_ptr(cc), dtype_code(cc.dtype), b, t, r, route_start, route_end, _orders(orders),
                               len(orders), bits, _ptr(seg), _ptr(val), _ptr(out), dtype_code(rows_dtype),
                               _stream(dev)), "ngram_rows")
    return out


def online_mix(keys: torch.Tensor, nxt: torch.Tensor, q: torch.Tensor, deadline: torch.Tensor, p: torch.Tensor,
               kappa: float = 1.0) -> torch.Tensor:
    """``OnlineCounts.mix`` (``drafting/drafters.py:117-142``): keys ``[T, R, n_orders]`` int32 rows of
    the committed pairs, ``nxt [T]`` their next tokens, q ``[N, R, n_orders]`` int32 query rows,
    ``deadline [N]``, p ``[N, V]`` fp32 -> the mixed ``[N, V]`` fp32."""
    dev = _dev(keys, nxt, q, deadline, p)
    t, r, no = keys.shape
    n, v = p.shape
    if q.shape != (n, r, no) or nxt.shape != (t,) or deadline.shape != (n,):
        raise ValueError("online_mix: keys [T, R, n], nxt [T], q [N, R, n], deadline [N], p [N, V]")
    kc, qc = _c(keys.to(torch.int32)), _c(q.to(torch.int32))
    xc, dc, pc = _c(nxt.to(torch.int64)), _c(deadline.to(torch.int64)), _c(p.to(torch.float32))
    work = torch.empty(max(n * t, 1), dtype=torch.float32, device=dev)
    out = torch.empty(n, v, dtype=torch.float32, device=dev)
    check(lib().lng_online_mix(_ptr(kc), _ptr(xc), t, _ptr(qc), _ptr(dc), n, r, no, _ptr(pc), v, float(kappa),
                               _ptr(work), _ptr(out), _stream(dev)), "online_mix")
    return out


def route_tokens(codes: torch.Tensor, tables, orders, bits: int, route_start: int = 0, route_end: int | None = None,
                 segment_ids=None, valid_tokens=None, target_length: int | None = None) -> torch.Tensor:
    """Route tokens ``[B, T_out, R', len(orders)*mem_dim]`` gathered from ``tables`` (one per order)."""
    dev = _dev(codes, *tables, segment_ids, valid_tokens)
    b, t, r = codes.shape
    route_end = r if route_end is None else route_end
    tabs = [_c(tb) for tb in tables]
    dt = tabs[0].dtype
    mem_dim = tabs[0].shape[1]
    for tb in tabs:
        if tb.dtype != dt or tb.shape[1] != mem_dim:
            raise ValueError("all n-gram tables must share dtype and width")
    cc = _codes_ok(codes)
    seg, val = _seg(segment_ids, valid_tokens)
    t_out = t if not target_length else int(target_length)
    out = torch.empty(b, t_out, route_end - route_start, len(orders) * mem_dim, dtype=dt, device=dev)
    tp = (ctypes.c_void_p * len(tabs))(*[tb.data_ptr() for tb in tabs])
    check(lib().lng_route_tokens(_ptr(cc), dtype_code(cc.dtype), b, t, r, route_start, route_end, _orders(orders),
                                 len(orders), bits, tp, dtype_code(dt), mem_dim, _ptr(seg), _ptr(val),
                                 int(target_length or 0), _ptr(out), _stream(dev)), "route_tokens")
    return out


# ----------------------------------------------------------------------------- K3 pieces
def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, fused: bool = False) -> torch.Tensor:
    """RMSNorm over the last dim.  ``fused=False``: ``model.RMSNorm`` (``model.py:39-48``: round the
    normalised row, multiply by the weight, round); ``fused=True``: ``lngram_v2.RMSNorm``
    (``lngram_v2.py:36-53``, ``F.rms_norm``: weight applied in fp32, one rounding)."""
    dev = _dev(x, w)
    xc = _c(x)
    wc = _c(w.to(x.dtype))
    out = torch.empty_like(xc)
    d = x.shape[-1]
    mode = _lib.NORM_FUSED if fused else _lib.NORM_MODEL
    check(lib().lng_rmsnorm(_ptr(xc), _ptr(wc), dtype_code(x.dtype), xc.numel() // d, d, eps, mode, _ptr(out),
                            _stream(dev)), "rmsnorm")
    return out


def linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """``x [..., K] . w[N, K]^T`` in x's dtype (fp32 accumulation)."""
    dev = _dev(x, w)
    k = x.shape[-1]
    x2 = _c(x.reshape(-1, k))
    wc = _c(w.to(x.dtype))
    n = wc.shape[0]
    if wc.shape[1] != k:
        raise ValueError(f"weight {tuple(w.shape)} does not match input dim {k}")
    out = torch.empty(*x.shape[:-1], n, dtype=x.dtype, device=dev)
    check(lib().lng_linear(_ptr(x2), _ptr(wc), dtype_code(x.dtype), x2.shape[0], n, k, _ptr(out), _stream(dev)),
          "linear")
    return out


def linear_rowscale_ok(x: torch.Tensor, w: torch.Tensor) -> bool:
    """Whether :func:`linear_rowscale` serves this bf16 shape (``lng_linear_rowscale_ok``)."""
    k = x.shape[-1]
    return (x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and w.dim() == 2 and w.shape[1] == k
            and bool(lib().lng_linear_rowscale_ok(x.numel() // k, w.shape[0], k)))


def linear_rowscale(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """bf16 ``(x . w^T) * rsqrt(mean(x^2, -1) + eps)`` per row (``lng_linear_rowscale``): the projection
    of ``RMSNorm(x)`` with the norm's weight folded into ``w``, the row scale formed inside the GEMM."""
    dev = _dev(x, w)
    k = x.shape[-1]
    x2 = _c(x.reshape(-1, k))
    wc = _c(w)
    if x.dtype != torch.bfloat16 or wc.dtype != torch.bfloat16 or wc.shape[1] != k:
        raise ValueError("linear_rowscale needs bf16 x [..., K] and w [N, K]")
    n = wc.shape[0]
    out = torch.empty(*x.shape[:-1], n, dtype=x.dtype, device=dev)
    check(lib().lng_linear_rowscale(_ptr(x2), _ptr(wc), x2.shape[0], n, k, float(eps), _ptr(out), _stream(dev)),
          "linear_rowscale")
    return out


def _at_args(cache: torch.Tensor, pos0_dev: torch.Tensor | None):
    if cache.dim() != 3 or not cache.is_contiguous():
        raise ValueError("the cache must be a contiguous [B, S, N] tensor")
    if pos0_dev is not None and (pos0_dev.dtype != torch.int32 or pos0_dev.numel() != 1):
        raise ValueError("pos0_dev must be one int32 on the device")


def linear_at(x: torch.Tensor, w: torch.Tensor, cache: torch.Tensor, pos0: int = 0,
              pos0_dev: torch.Tensor | None = None) -> None:
    """bf16 ``x [B, n, K] . w[N, K]^T`` written into ``cache [B, S, N]`` at positions
    ``p0 .. p0+n-1``, ``p0 = pos0 (+ pos0_dev)`` (``lng_linear_at``; B*n <= 64)."""
    dev = _dev(x, w, cache, pos0_dev)
    _at_args(cache, pos0_dev)
    b, n, k = x.shape
    xc, wc = _c(x), _c(w.to(x.dtype))
    if x.dtype != torch.bfloat16 or cache.dtype != torch.bfloat16 or cache.shape[0] != b or cache.shape[2] != wc.shape[0]:
        raise ValueError("linear_at: bf16 x [B, n, K] and cache [B, S, N]")
    check(lib().lng_linear_at(_ptr(xc), _ptr(wc), b * n, wc.shape[0], k, n, cache.shape[1], int(pos0), _ptr(pos0_dev),
                              _ptr(cache), _stream(dev)), "linear_at")


def router_codes_at(x: torch.Tensor, w: torch.Tensor, cache: torch.Tensor, pos0: int = 0,
                    pos0_dev: torch.Tensor | None = None) -> None:
    """4-bit route codes of bf16 ``x [B, n, K] . w[4R, K]^T`` written into the uint8 code cache
    ``[B, S, R]`` at positions ``p0 .. p0+n-1`` (``lng_router_codes_at``; B*n <= 64)."""
    dev = _dev(x, w, cache, pos0_dev)
    _at_args(cache, pos0_dev)
    b, n, k = x.shape
    xc, wc = _c(x), _c(w)
    if (x.dtype != torch.bfloat16 or wc.dtype != torch.bfloat16 or cache.dtype != torch.uint8
            or cache.shape[0] != b or 4 * cache.shape[2] != wc.shape[0]):
        raise ValueError("router_codes_at: bf16 x [B, n, K], router [4R, K], uint8 cache [B, S, R]")
    check(lib().lng_router_codes_at(_ptr(xc), _ptr(wc), b * n, k, wc.shape[0], n, cache.shape[1], int(pos0),
                                    _ptr(pos0_dev), _ptr(cache), _stream(dev)), "router_codes_at")


def tree_windows(cache: torch.Tensor, node_codes: torch.Tensor, idx: torch.Tensor, hist: int, L: int,
                 L_dev: torch.Tensor | None, rel: torch.Tensor):
    """The n-gram windows of a draft tree's nodes and the node codes cached (``lng_tree_windows``):
    ``cache [B, max_len, R]`` u8 (written at ``L .. L+n-1``), ``node_codes [B, n, R]``, ``idx
    [n, hist+1]`` and ``rel [n, k]`` int32 device tables, ``L_dev`` a device int32 added to ``L``.
    Returns ``(win [B*n, hist+1, R] u8, seg int32, val u8 [B*n, hist+1], slots [n, k] int32)``."""
    dev = _dev(cache, node_codes, idx, rel, L_dev)
    if cache.dtype != torch.uint8 or not cache.is_contiguous() or cache.dim() != 3:
        raise ValueError("tree_windows: cache must be a contiguous [B, max_len, R] uint8 tensor")
    b, max_len, r = cache.shape
    nc = _c(node_codes)
    n = nc.shape[1]
    if tuple(nc.shape) != (b, n, r) or idx.dtype != torch.int32 or rel.dtype != torch.int32:
        raise ValueError("tree_windows: node codes [B, n, R], int32 idx and rel")
    h1 = idx.shape[1]
    win = torch.empty(b * n, h1, r, dtype=torch.uint8, device=dev)
    seg = torch.empty(b * n, h1, dtype=torch.int32, device=dev)
    val = torch.empty(b * n, h1, dtype=torch.uint8, device=dev)
    slots = torch.empty(n, rel.shape[1], dtype=torch.int32, device=dev)
    check(lib().lng_tree_windows(_ptr(nc), dtype_code(nc.dtype), _ptr(cache), b, max_len, r, n, int(hist),
                                 _ptr(_c(idx)), int(L), _ptr(L_dev), _ptr(_c(rel)), rel.shape[1], _ptr(win),
                                 _ptr(seg), _ptr(val), _ptr(slots), _stream(dev)), "tree_windows")
    return win, seg, val, slots


def linear_rowsq(x: torch.Tensor, w: torch.Tensor):
    """bf16 ``x [..., K] . w[N, K]^T`` plus the partial row sums of squares of the bf16 output
    (``[P, rows]`` fp32) that :func:`causal_conv_rowsq` consumes."""
    dev = _dev(x, w)
    k = x.shape[-1]
    x2 = _c(x.reshape(-1, k))
    wc = _c(w.to(x.dtype))
    n = wc.shape[0]
    if x.dtype != torch.bfloat16 or k % 32:
        raise ValueError("linear_rowsq needs bf16 operands and K % 32 == 0")
    p = int(lib().lng_linear_rowsq_partials(n))
    out = torch.empty(*x.shape[:-1], n, dtype=x.dtype, device=dev)
    rowsq = torch.empty(p, x2.shape[0], dtype=torch.float32, device=dev)
    rc = _timed("linear", dev, lambda: lib().lng_linear_rowsq(_ptr(x2), _ptr(wc), x2.shape[0], n, k, _ptr(out),
                                                                _ptr(rowsq), _stream(dev)))
    check(rc, "linear_rowsq")
    return out, rowsq


def row_sumsq(x: torch.Tensor) -> torch.Tensor:
    """``[1, rows]`` fp32 sums of squares of the bf16 rows of ``x`` (the layout of
    :func:`linear_rowsq`'s statistics with one partial)."""
    dev = _dev(x)
    if x.dtype != torch.bfloat16:
        raise ValueError("row_sumsq needs bf16 rows")
    d = x.shape[-1]
    xc = _c(x.reshape(-1, d))
    out = torch.empty(1, xc.shape[0], dtype=torch.float32, device=dev)
    check(lib().lng_row_sumsq(_ptr(xc), xc.shape[0], d, _ptr(out), _stream(dev)), "row_sumsq")
    return out


def causal_conv_rowsq(mixed: torch.Tensor, rowsq: torch.Tensor, norm_w: torch.Tensor, conv_w: torch.Tensor,
                      dilation: int, eps: float, residual: bool = True) -> torch.Tensor:
    """:func:`causal_conv` (bf16, kernel 4, dilation 3) with row statistics from :func:`linear_rowsq`."""
    dev = _dev(mixed, rowsq, norm_w, conv_w)
    m = _c(mixed)
    b, t, d = m.shape
    cw = _c(conv_w.reshape(d, -1).to(m.dtype))
    nw = _c(norm_w.to(m.dtype))
    rs = _c(rowsq)
    out = torch.empty_like(m)
    rc = _timed("causal_conv", dev, lambda: lib().lng_causal_conv_rowsq(
        _ptr(m), _ptr(rs), rs.shape[0], _ptr(nw), _ptr(cw), b, t, d, cw.shape[1], dilation, eps, int(bool(residual)),
        _ptr(out), _stream(dev)))
    check(rc, "causal_conv_rowsq")
    return out


def sink_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, scale: float,
                   sink_logit: float) -> torch.Tensor:
    """query ``[B, T, KV, G, hd]``; key/value ``[B, T, KV, R, hd]`` (head dim contiguous, any other
    strides) -> ``[B, T, KV, G, hd]``."""
    dev = _dev(query, key, value)
    b, t, kv, g, hd = query.shape
    r = key.shape[3]
    q = _c(query)
    if key.stride(-1) != 1:
        key = key.contiguous()
    if value.stride(-1) != 1:
        value = value.contiguous()
    if key.dtype != q.dtype or value.dtype != q.dtype:
        raise TypeError("query, key and value must share a dtype")

    def bt_strides(x):
        # (b, t) must collapse into one stride
        sb, st = x.stride(0), x.stride(1)
        if b > 1 and sb != st * t:
            return None
        return (st, x.stride(2), x.stride(3))

    ks, vs = bt_strides(key), bt_strides(value)
    if ks is None:
        key = key.contiguous()
        ks = bt_strides(key)
    if vs is None:
        value = value.contiguous()
        vs = bt_strides(value)
    out = torch.empty(b, t, kv, g, hd, dtype=q.dtype, device=dev)
    ka = (ctypes.c_int64 * 3)(*ks)
    va = (ctypes.c_int64 * 3)(*vs)
    check(lib().lng_sink_attention_strided(_ptr(q), ctypes.c_void_p(key.data_ptr()), ctypes.c_void_p(value.data_ptr()),
                                           dtype_code(q.dtype), b * t, kv, g, r, hd, ka, va, scale, sink_logit,
                                           _ptr(out), _stream(dev)), "sink_attention")
    return out


def sink_probabilities(scores: torch.Tensor, sink_logit: float) -> torch.Tensor:
    dev = _dev(scores)
    s = _c(scores.float())
    r = s.shape[-1]
    out = torch.empty_like(s)
    check(lib().lng_sink_probabilities(_ptr(s), s.numel() // r, r, sink_logit, _ptr(out), _stream(dev)),
          "sink_probabilities")
    return out


def causal_conv(mixed: torch.Tensor, norm_w: torch.Tensor, conv_w: torch.Tensor, dilation: int,
                eps: float, residual: bool = True) -> torch.Tensor:
    """``[mixed +] SiLU(conv(RMSNorm(mixed)))`` for mixed ``[B, T, d]``, conv weight ``[d, 1, K]``."""
    dev = _dev(mixed, norm_w, conv_w)
    m = _c(mixed)
    b, t, d = m.shape
    cw = _c(conv_w.reshape(d, -1).to(m.dtype))
    nw = _c(norm_w.to(m.dtype))
    out = torch.empty_like(m)
    check(lib().lng_causal_conv(_ptr(m), _ptr(nw), _ptr(cw), dtype_code(m.dtype), b, t, d, cw.shape[1], dilation,
                                eps, int(bool(residual)), _ptr(out), _stream(dev)), "causal_conv")
    return out


def causal_conv_at(rows: torch.Tensor, norm_w: torch.Tensor, conv_w: torch.Tensor, dilation: int, eps: float,
                   pos0: int, n: int, length: int | None = None, pos0_dev: torch.Tensor | None = None,
                   residual: bool = True) -> torch.Tensor:
    """``causal_conv`` for positions ``p0 .. p0+n-1`` of cached rows (``lng_causal_conv_at``):
    ``rows [B, S, d]`` hold the conv's (pre-norm) inputs of positions ``0 .. length-1`` (default
    ``length = S``); ``p0 = pos0 (+ pos0_dev)``, ``pos0_dev`` an int32 device scalar (the cached
    length read on the device, for launches captured in a graph) -> ``[B, n, d]``."""
    dev = _dev(rows, norm_w, conv_w, pos0_dev)
    if rows.dim() != 3 or rows.stride(-1) != 1 or rows.stride(1) != rows.shape[-1]:
        raise ValueError("causal_conv_at: rows must be [B, S, d] with contiguous rows")
    b, s_len, d = rows.shape
    length = s_len if length is None else int(length)
    cw = _c(conv_w.reshape(d, -1).to(rows.dtype))
    nw = _c(norm_w.to(rows.dtype))
    pd = None
    if pos0_dev is not None:
        if pos0_dev.dtype != torch.int32 or pos0_dev.numel() != 1:
            raise ValueError("causal_conv_at: pos0_dev must be one int32 on the device")
        pd = pos0_dev
    out = torch.empty(b, n, d, dtype=rows.dtype, device=dev)
    check(lib().lng_causal_conv_at(_ptr(rows), _ptr(nw), _ptr(cw), dtype_code(rows.dtype), b, rows.stride(0) // d,
                                   length, int(pos0), _ptr(pd), int(n), d, cw.shape[1], dilation, eps,
                                   int(bool(residual)), _ptr(out), _stream(dev)), "causal_conv_at")
    return out


def causal_conv_slots(rows: torch.Tensor, norm_w: torch.Tensor, conv_w: torch.Tensor, dilation: int, eps: float,
                      slots: torch.Tensor, length: int | None = None, residual: bool = True) -> torch.Tensor:
    """The short conv with each output's window given as cache rows (``lng_causal_conv_slots``):
    ``slots [n, back + 1]`` (oldest first, ``back = (K - 1) * dilation``; the ancestor windows of
    ``tree_slots``) index the rows ``[B, S, d]`` of every sequence; a slot outside ``[0, length)``
    (default ``length = S``) is a zero row.  Output ``i`` also adds row ``slots[i, back]`` as the
    residual -> ``[B, n, d]``."""
    dev = _dev(rows, norm_w, conv_w)
    if rows.dim() != 3 or rows.stride(-1) != 1 or rows.stride(1) != rows.shape[-1]:
        raise ValueError("causal_conv_slots: rows must be [B, S, d] with contiguous rows")
    b, s_len, d = rows.shape
    length = s_len if length is None else int(length)
    cw = _c(conv_w.reshape(d, -1).to(rows.dtype))
    k = cw.shape[1]
    back = (k - 1) * int(dilation)
    sl = _c(slots.to(device=dev, dtype=torch.int32))
    if sl.dim() != 2 or sl.shape[1] != back + 1:
        raise ValueError(f"causal_conv_slots: slots must be [n, {back + 1}]")
    nw = _c(norm_w.to(rows.dtype))
    n = sl.shape[0]
    out = torch.empty(b, n, d, dtype=rows.dtype, device=dev)
    check(lib().lng_causal_conv_slots(_ptr(rows), _ptr(nw), _ptr(cw), dtype_code(rows.dtype), b, rows.stride(0) // d,
                                      length, _ptr(sl), n, back, d, k, int(dilation), eps, int(bool(residual)),
                                      _ptr(out), _stream(dev)), "causal_conv_slots")
    return out


def memory_readout_pack(kv: torch.Tensor) -> torch.Tensor:
    """``readout_kv_proj.weight`` ``[512, 256]`` bf16 -> the fused readout's packed KV weight
    (``lng_memory_readout_pack``: a permutation into the kernel's operand order)."""
    dev = _dev(kv)
    kc = _c(kv)
    if kc.dtype != torch.bfloat16 or kc.shape != (512, 256):
        raise ValueError("fused readout packs a bf16 [512, 256] kv_proj weight")
    out = torch.empty(_lib.READOUT_PACK_ELEMS, dtype=torch.bfloat16, device=dev)
    check(lib().lng_memory_readout_pack(_ptr(kc), _ptr(out), _stream(dev)), "memory_readout_pack")
    return out


def fold_columns(w: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """``w[N, K] * s[K]`` in bf16 (one rounding): a row RMSNorm's weight folded into the projection after it."""
    dev = _dev(w, s)
    wc, sc = _c(w.to(torch.bfloat16)), _c(s.to(torch.bfloat16))
    n, k = wc.shape
    if sc.shape != (k,):
        raise ValueError("fold_columns: w [N, K], s [K]")
    out = torch.empty_like(wc)
    check(lib().lng_fold_columns(_ptr(wc), _ptr(sc), n, k, _ptr(out), _stream(dev)), "fold_columns")
    return out


def memory_readout_fused(q: torch.Tensor, codes: torch.Tensor, table2: torch.Tensor, table3: torch.Tensor,
                         kv_pack: torch.Tensor, w_mem: torch.Tensor, eps: float, scale: float,
                         sink_logit: float, q_rows: torch.Tensor | None = None, q_eps: float = 0.0) -> torch.Tensor:
    """Fused gather + sink readout (bf16, 16 heads x 64, 4 KV heads, orders (2,3), mem_dim 128).

    q ``[B, T, 1024]``, codes ``[B, T, R]`` uint8, ``kv_pack`` from ``memory_readout_pack`` ->
    head output ``[B, T, 1024]``.  With ``q_rows [B, T, 1024]`` (the projection's input rows; q was
    projected with the query RMSNorm's weight folded in), each token's query is scaled by its row's
    ``rsqrt(mean(row^2) + q_eps)`` inside the kernel."""
    dev = _dev(q, codes, table2, table3, kv_pack, w_mem, q_rows)
    b, t, r = codes.shape
    qc = _c(q)
    cc = _c(codes.to(torch.uint8))
    if qc.dtype != torch.bfloat16 or qc.shape[-1] != 1024:
        raise ValueError("fused readout expects a bf16 [B, T, 1024] query")
    if table2.shape != (r * 256, 128) or table3.shape != (r * 4096, 128):
        raise ValueError("fused readout expects tables [R*256,128] and [R*4096,128]")
    if kv_pack.shape != (_lib.READOUT_PACK_ELEMS,) or kv_pack.dtype != torch.bfloat16 or w_mem.shape != (256,):
        raise ValueError("fused readout weight shapes")
    qr = None
    if q_rows is not None:
        qr = _c(q_rows)
        if qr.dtype != torch.bfloat16 or qr.shape != qc.shape:
            raise ValueError("fused readout: q_rows must be bf16 and shaped like q")
    out = torch.empty(b, t, 1024, dtype=torch.bfloat16, device=dev)
    t2, t3, kp, wmc = _c(table2), _c(table3), _c(kv_pack), _c(w_mem.to(torch.bfloat16))
    rc = _timed("memory_readout_fused", dev, lambda: lib().lng_memory_readout_fused(
        _ptr(qc), _ptr(qr), float(q_eps), _ptr(cc), b, t, r, _ptr(t2), _ptr(t3), _ptr(kp), _ptr(wmc), eps, scale,
        sink_logit, _ptr(out), _stream(dev)))
    check(rc, "memory_readout_fused")
    return out


def memory_readout_fused_at(q: torch.Tensor, codes: torch.Tensor, pos0: int, table2: torch.Tensor,
                            table3: torch.Tensor, kv_pack: torch.Tensor, w_mem: torch.Tensor, eps: float,
                            scale: float, sink_logit: float, q_rows: torch.Tensor | None = None, q_eps: float = 0.0,
                            pos0_dev: torch.Tensor | None = None) -> torch.Tensor:
    """``memory_readout_fused`` for ``n`` new positions (``lng_memory_readout_fused_at``): q
    ``[B, n, 1024]``; codes ``[B, S, R]`` uint8 (a code cache or a verification context, row stride
    ``S * R``) with the new tokens at positions ``p0 .. p0+n-1``, ``p0 = pos0 (+ pos0_dev)``."""
    dev = _dev(q, codes, table2, table3, kv_pack, w_mem, q_rows, pos0_dev)
    b, n = q.shape[0], q.shape[1]
    if codes.dim() != 3 or codes.dtype != torch.uint8 or codes.shape[0] != b or not codes.is_contiguous():
        raise ValueError("fused readout: codes must be a contiguous uint8 [B, S, R] cache")
    r = codes.shape[2]
    qc = _c(q)
    if qc.dtype != torch.bfloat16 or qc.shape[-1] != 1024:
        raise ValueError("fused readout expects a bf16 [B, n, 1024] query")
    if table2.shape != (r * 256, 128) or table3.shape != (r * 4096, 128):
        raise ValueError("fused readout expects tables [R*256,128] and [R*4096,128]")
    if kv_pack.shape != (_lib.READOUT_PACK_ELEMS,) or kv_pack.dtype != torch.bfloat16 or w_mem.shape != (256,):
        raise ValueError("fused readout weight shapes")
    qr = None
    if q_rows is not None:
        qr = _c(q_rows)
        if qr.dtype != torch.bfloat16 or qr.shape != qc.shape:
            raise ValueError("fused readout: q_rows must be bf16 and shaped like q")
    if pos0_dev is not None and (pos0_dev.dtype != torch.int32 or pos0_dev.numel() != 1):
        raise ValueError("fused readout: pos0_dev must be one int32 on the device")
    out = torch.empty(b, n, 1024, dtype=torch.bfloat16, device=dev)
    t2, t3, kp, wmc = _c(table2), _c(table3), _c(kv_pack), _c(w_mem.to(torch.bfloat16))
    check(lib().lng_memory_readout_fused_at(_ptr(qc), _ptr(qr), float(q_eps), _ptr(codes), b, n, r, codes.shape[1],
                                            int(pos0), _ptr(pos0_dev), _ptr(t2), _ptr(t3), _ptr(kp), _ptr(wmc), eps,
                                            scale, sink_logit, _ptr(out), _stream(dev)), "memory_readout_fused_at")
    return out


def memory_readout_fused_rows(q: torch.Tensor, route_tokens: torch.Tensor, kv_pack: torch.Tensor, w_mem: torch.Tensor,
                              eps: float, scale: float, sink_logit: float, q_rows: torch.Tensor | None = None,
                              q_eps: float = 0.0) -> torch.Tensor:
    """The fused readout over supplied route tokens (``lng_memory_readout_fused_rows``): q ``[B, n,
    1024]``, route_tokens ``[B, n, R, 256]`` bf16 -> head ``[B, n, 1024]``, equal to the code path's
    output for the same rows."""
    dev = _dev(q, route_tokens, kv_pack, w_mem, q_rows)
    b, n = q.shape[0], q.shape[1]
    if route_tokens.dim() != 4 or route_tokens.shape[:2] != (b, n) or route_tokens.shape[3] != 256 or \
            route_tokens.dtype != torch.bfloat16:
        raise ValueError("fused readout: route tokens must be bf16 [B, n, R, 256]")
    r = route_tokens.shape[2]
    qc, rt = _c(q), _c(route_tokens)
    if qc.dtype != torch.bfloat16 or qc.shape[-1] != 1024:
        raise ValueError("fused readout expects a bf16 [B, n, 1024] query")
    if kv_pack.shape != (_lib.READOUT_PACK_ELEMS,) or kv_pack.dtype != torch.bfloat16 or w_mem.shape != (256,):
        raise ValueError("fused readout weight shapes")
    qr = None
    if q_rows is not None:
        qr = _c(q_rows)
        if qr.dtype != torch.bfloat16 or qr.shape != qc.shape:
            raise ValueError("fused readout: q_rows must be bf16 and shaped like q")
    out = torch.empty(b, n, 1024, dtype=torch.bfloat16, device=dev)
    kp, wmc = _c(kv_pack), _c(w_mem.to(torch.bfloat16))
    check(lib().lng_memory_readout_fused_rows(_ptr(qc), _ptr(qr), float(q_eps), _ptr(rt), b, n, r, _ptr(kp), _ptr(wmc),
                                              eps, scale, sink_logit, _ptr(out), _stream(dev)),
          "memory_readout_fused_rows")
    return out


def gather_sum_scaled(tables, codes: torch.Tensor, orders, bits: int, scale_log2: int, seed: int) -> torch.Tensor:
    """fp32 ``[B, T, mem_dim]``: per token, the sum of one row per (route, order) of tables grown
    ``2**scale_log2`` times per route (``lng_gather_sum_scaled``); ``codes [B, T, R]`` uint8,
    ``tables[i]`` ``[R * 2**scale_log2 * 2**(bits * orders[i]), mem_dim]`` bf16 or fp32."""
    dev = _dev(codes, *tables)
    b, t, r = codes.shape
    tabs = [_c(tb) for tb in tables]
    dt = tabs[0].dtype
    md = tabs[0].shape[1]
    if len(tabs) != len(orders):
        raise ValueError("one table per order")
    for tb, n in zip(tabs, orders):
        if tb.dtype != dt or tb.shape != (r << (int(scale_log2) + bits * int(n)), md):
            raise ValueError(f"table of order {n} must be [R * 2^scale_log2 * 2^(bits n), mem_dim] = "
                             f"[{r << (int(scale_log2) + bits * int(n))}, {md}] {dt}, got {tuple(tb.shape)} {tb.dtype}")
    cc = _c(codes.to(torch.uint8))
    out = torch.empty(b, t, md, dtype=torch.float32, device=dev)
    tp = (ctypes.c_void_p * len(tabs))(*[tb.data_ptr() for tb in tabs])
    rc = _timed("gather_sum_scaled", dev, lambda: lib().lng_gather_sum_scaled(
        tp, dtype_code(dt), md, _ptr(cc), b, t, r, _orders(orders), len(orders), bits, int(scale_log2),
        ctypes.c_uint32(int(seed) & 0xFFFFFFFF), _ptr(out), _stream(dev)))
    check(rc, "gather_sum_scaled")
    return out


_sg_ws: dict = {}
_sg_ws_lock = threading.Lock()


def _surrogate_workspace(dev: torch.device, nbytes: int) -> torch.Tensor:
    """Scratch of ``lng_surrogate_grad_ws`` for (device, current stream), grown as needed: a call writes
    every byte of it that it reads, and calls on one stream run in order."""
    key = (dev.index, torch.cuda.current_stream(dev).cuda_stream)
    with _sg_ws_lock:
        ws = _sg_ws.get(key)
        if ws is None or ws.numel() < nbytes:
            ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
            _sg_ws[key] = ws
        return ws


def surrogate_grad(grad_memory: torch.Tensor, hard_memory: torch.Tensor | None, q_logits: torch.Tensor,
                   codes: torch.Tensor, table: torch.Tensor, valid_mask: torch.Tensor | None, order: int, bits: int,
                   route_start: int, temperature: float, scale: float, exact: bool,
                   workspace: bool = True) -> torch.Tensor:
    """Route-logit gradient ``[B, T, R, bits]`` (``q_logits``' dtype) of the lookup surrogate of one
    order (``lng_surrogate_grad``; ``_LngramSurrogate.backward``, ``lngram_v2.py:364-464``).
    ``hard_memory`` None: it is the lookup's own rows (``table[row] * valid``), which the kernel
    then reads from the table instead of streaming them.  ``workspace``: shapes that have a
    workspace path (``lng_surrogate_workspace_bytes``) take it (``lng_surrogate_grad_ws``)."""
    dev = _dev(grad_memory, hard_memory, q_logits, codes, table, valid_mask)
    b, t, r, md = grad_memory.shape
    if (hard_memory is not None and tuple(hard_memory.shape) != (b, t, r, md)) or \
            tuple(q_logits.shape) != (b, t, r, bits) or tuple(codes.shape) != (b, t, r) or table.dim() != 2 or \
            table.shape[1] != md:
        raise ValueError("surrogate_grad: memory [B,T,R,D], q_logits [B,T,R,bits], codes [B,T,R], table [rows, D]")
    mdt = table.dtype
    if hard_memory is not None and hard_memory.dtype != mdt:
        raise ValueError(f"surrogate_grad: memory dtype {hard_memory.dtype} != table dtype {mdt}")
    g = _c(grad_memory.to(mdt))
    hm, tab, q, cc = _c(hard_memory), _c(table), _c(q_logits), _c(codes)
    if cc.dtype not in (torch.uint8, torch.int32, torch.int64):
        cc = _c(cc.to(torch.int64))
    vm = None if valid_mask is None else _c(valid_mask.to(torch.uint8))
    if vm is not None and tuple(vm.shape) != (b, t):
        raise ValueError("surrogate_grad: valid_mask must be [B, T]")
    out = torch.empty(b, t, r, bits, dtype=q.dtype, device=dev)
    nws = lib().lng_surrogate_workspace_bytes(b, t, r, md, int(order), int(bits), dtype_code(mdt),
                                              int(bool(exact))) if workspace else 0
    if nws:
        ws = _surrogate_workspace(dev, nws)
        rc = _timed("surrogate_grad", dev, lambda: lib().lng_surrogate_grad_ws(
            _ptr(g), _ptr(hm), dtype_code(mdt), _ptr(q), dtype_code(q.dtype), _ptr(cc), dtype_code(cc.dtype),
            _ptr(tab), tab.shape[0], _ptr(vm), b, t, r, int(route_start), md, int(order), int(bits),
            float(temperature), float(scale), int(bool(exact)), _ptr(ws), ws.numel(), _ptr(out),
            dtype_code(out.dtype), _stream(dev)))
    else:
        rc = _timed("surrogate_grad", dev, lambda: lib().lng_surrogate_grad(
            _ptr(g), _ptr(hm), dtype_code(mdt), _ptr(q), dtype_code(q.dtype), _ptr(cc), dtype_code(cc.dtype),
            _ptr(tab), tab.shape[0], _ptr(vm), b, t, r, int(route_start), md, int(order), int(bits),
            float(temperature), float(scale), int(bool(exact)), _ptr(out), dtype_code(out.dtype), _stream(dev)))
    check(rc, "surrogate_grad")
    return out


def table_grad(grad_memory: torch.Tensor, codes: torch.Tensor, valid_mask: torch.Tensor | None, order: int,
               bits: int, route_start: int, table_rows: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 ``[table_rows, D]`` table gradient of one order's lookup (``lng_table_grad``): the
    embedding backward of ``_lookup_route_chunk``'s gather; adds into ``out`` when given."""
    dev = _dev(grad_memory, codes, valid_mask, out)
    b, t, r, md = grad_memory.shape
    if tuple(codes.shape) != (b, t, r):
        raise ValueError("table_grad: codes must be [B, T, R]")
    g = _c(grad_memory if grad_memory.dtype in (torch.float32, torch.bfloat16) else grad_memory.float())
    cc = _c(codes if codes.dtype in (torch.uint8, torch.int32, torch.int64) else codes.to(torch.int64))
    vm = None if valid_mask is None else _c(valid_mask.to(torch.uint8))
    if out is None:
        out = torch.zeros(int(table_rows), md, dtype=torch.float32, device=dev)
    elif out.dtype != torch.float32 or tuple(out.shape) != (int(table_rows), md) or not out.is_contiguous():
        raise ValueError("table_grad: out must be a contiguous fp32 [table_rows, D]")
    rc = _timed("table_grad", dev, lambda: lib().lng_table_grad(
        _ptr(g), dtype_code(g.dtype), _ptr(cc), dtype_code(cc.dtype), _ptr(vm), b, t, r, int(route_start), md,
        int(order), int(bits), int(table_rows), _ptr(out), _stream(dev)))
    check(rc, "table_grad")
    return out


# ----------------------------------------------------------------------------- serving layout
def table_address(t: torch.Tensor) -> int:
    """Device-visible address of a table's first element: a GPU tensor's own, or the mapping of a
    pinned host tensor into the device's address space (``lng_host_device_pointer``), through which
    the serving kernels read host RAM directly."""
    if t.device.type == "cuda":
        return t.data_ptr()
    if t.device.type != "cpu" or not t.is_pinned():
        raise RuntimeError("a host table must be pinned host memory (allocate it with pin_memory=True)")
    base = t.untyped_storage().data_ptr()
    dp = ctypes.c_void_p()
    check(lib().lng_host_device_pointer(ctypes.c_void_p(base), ctypes.byref(dp)), "host_device_pointer")
    return dp.value + (t.data_ptr() - base)


def _table_args(tables, orders, bits: int, routes: int):
    ts = [t if t.is_contiguous() else None for t in tables]
    if any(t is None for t in ts):
        raise ValueError("serving tables must be contiguous")
    dt, md = ts[0].dtype, ts[0].shape[1]
    for t, o in zip(ts, orders):
        if t.dtype != dt or t.dim() != 2 or t.shape[1] != md:
            raise ValueError("serving tables: one dtype and row width")
        if t.shape[0] < routes << (bits * int(o)):
            raise ValueError(f"serving table of order {o} has {t.shape[0]} rows, needs {routes << (bits * int(o))}")
    ptrs = (ctypes.c_void_p * len(ts))(*[table_address(t) for t in ts])
    rows = (ctypes.c_int64 * len(ts))(*[t.shape[0] for t in ts])
    return ptrs, rows, dt, md


def permute_table(weight: torch.Tensor, routes: int, order: int, bits: int, out: torch.Tensor | None = None):
    """Serving layout of a v2 table, or back (an involution): ``lng_permute_table``."""
    dev = _dev(weight, out)
    w = _c(weight)
    if w.dim() != 2 or w.shape[0] != routes << (bits * order):
        raise ValueError(f"table must be [routes * 2^(bits*order), D], got {tuple(w.shape)}")
    out = torch.empty_like(w) if out is None else out
    if out.shape != w.shape or out.dtype != w.dtype or not out.is_contiguous():
        raise ValueError("permute_table: out must match the table")
    check(lib().lng_permute_table(_ptr(w), _ptr(out), dtype_code(w.dtype), int(routes), int(order), int(bits),
                                  w.shape[1], _stream(dev)), "permute_table")
    return out


def serving_address(codes: torch.Tensor, order: int, bits: int) -> torch.Tensor:
    """int64 ``[B, T-order+1, R]``: window addresses with the current code least significant."""
    dev = _dev(codes)
    c = _c(codes if codes.dtype in (torch.uint8, torch.int32, torch.int64) else codes.to(torch.int64))
    b, t, r = c.shape
    out = torch.empty(b, max(0, t - order + 1), r, dtype=torch.int64, device=dev)
    check(lib().lng_serving_address(_ptr(c), dtype_code(c.dtype), b, t, r, int(order), int(bits), _ptr(out),
                                    _stream(dev)), "serving_address")
    return out


def serving_gather(tables, orders, bits: int, ctx: torch.Tensor, n: int, start: int,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """Route tokens ``[B, n, R, len(orders) * D]`` of the last ``n`` positions of ``ctx [B, h + n, R]``
    (first new position = absolute ``start``) from serving-layout tables (device or pinned host
    memory): ``lng_serving_gather``."""
    dev = _dev(ctx, out)
    c = _c(ctx if ctx.dtype in (torch.uint8, torch.int32, torch.int64) else ctx.to(torch.int64))
    b, tc, r = c.shape
    h = tc - n
    ptrs, rows, dt, md = _table_args(tables, orders, bits, r)
    if out is None:
        out = torch.empty(b, n, r, len(orders) * md, dtype=dt, device=dev)
    elif out.shape != (b, n, r, len(orders) * md) or out.dtype != dt or not out.is_contiguous():
        raise ValueError("serving_gather: out must be a contiguous [B, n, R, len(orders) * D] of the tables' dtype")
    rc = _timed("serving_gather", dev, lambda: lib().lng_serving_gather(
        ptrs, rows, dtype_code(dt), md, _orders(orders), len(orders), int(bits), _ptr(c), dtype_code(c.dtype), b, h, n,
        r, int(start), _ptr(out), _stream(dev)))
    check(rc, "serving_gather")
    return out


def serving_candidates(tables, orders, bits: int, hist: torch.Tensor, position: int,
                       out: torch.Tensor | None = None) -> torch.Tensor:
    """Candidate blocks ``[B, R, len(orders), 2^bits, D]`` of ``position`` from the codes ``hist [B, h, R]``
    ending at ``position - 1``: ``lng_serving_candidates``."""
    dev = _dev(hist, out)
    c = _c(hist if hist.dtype in (torch.uint8, torch.int32, torch.int64) else hist.to(torch.int64))
    b, h, r = c.shape
    ptrs, rows, dt, md = _table_args(tables, orders, bits, r)
    shape = (b, r, len(orders), 1 << bits, md)
    if out is None:
        out = torch.empty(shape, dtype=dt, device=dev)
    elif tuple(out.shape) != shape or out.dtype != dt or not out.is_contiguous():
        raise ValueError(f"serving_candidates: out must be a contiguous {shape} of the tables' dtype")
    rc = _timed("serving_candidates", dev, lambda: lib().lng_serving_candidates(
        ptrs, rows, dtype_code(dt), md, _orders(orders), len(orders), int(bits), _ptr(c), dtype_code(c.dtype), b, h, r,
        int(position), _ptr(out), _stream(dev)))
    check(rc, "serving_candidates")
    return out


def gather_rows(table: torch.Tensor, idx: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``table[idx]`` (``[*idx.shape, D]``) by the device, from a device or pinned host table
    (``lng_gather_rows``); an index outside the table gives a zero row."""
    dev = _dev(idx, out)
    if table.dim() != 2 or not table.is_contiguous():
        raise ValueError("gather_rows: a contiguous [rows, D] table")
    ii = _c(idx.reshape(-1).to(torch.int64))
    md = table.shape[1]
    if out is None:
        out = torch.empty(ii.numel(), md, dtype=table.dtype, device=dev)
    elif out.numel() != ii.numel() * md or out.dtype != table.dtype or not out.is_contiguous():
        raise ValueError("gather_rows: out must be a contiguous buffer of idx.numel() rows")
    check(lib().lng_gather_rows(ctypes.c_void_p(table_address(table)), table.shape[0], dtype_code(table.dtype), md,
                                _ptr(ii), ii.numel(), _ptr(out), _stream(dev)), "gather_rows")
    return out.view(*idx.shape, md)


def select_candidates(cand: torch.Tensor, codes: torch.Tensor, bits: int) -> torch.Tensor:
    """``[M, R, K * D]`` rows of ``cand [M, R, K, 2^bits, D]`` at ``codes [M, R]``: ``lng_select_candidates``."""
    dev = _dev(cand, codes)
    cd = _c(cand)
    m, r, k, a, md = cd.shape
    if a != 1 << bits or tuple(codes.shape) != (m, r):
        raise ValueError("select_candidates: cand [M, R, K, 2^bits, D] and codes [M, R]")
    cc = _c(codes if codes.dtype in (torch.uint8, torch.int32, torch.int64) else codes.to(torch.int64))
    out = torch.empty(m, r, k * md, dtype=cd.dtype, device=dev)
    check(lib().lng_select_candidates(_ptr(cd), dtype_code(cd.dtype), md, _ptr(cc), dtype_code(cc.dtype), m, r, k,
                                      int(bits), _ptr(out), _stream(dev)), "select_candidates")
    return out


# ----------------------------------------------------------------------------- K4
_ssm_ws: dict = {}
_ssm_ws_lock = threading.Lock()


def _ssm_workspace(dev: torch.device, nbytes: int) -> torch.Tensor:
    """The scan's hand-off workspace for (device, current stream): zeroed once when it is made or
    grown, then reused (the kernel keeps its epoch in the workspace's header)."""
    key = (dev.index, torch.cuda.current_stream(dev).cuda_stream)
    with _ssm_ws_lock:
        ws = _ssm_ws.get(key)
        if ws is None or ws.numel() < nbytes:
            ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
        _ssm_ws[key] = ws
        return ws


def ssm_scan(a: torch.Tensor, u: torch.Tensor, s0: torch.Tensor | None = None,
             spin_limit: int | None = None, want_bf16: bool = False):
    """``s_t = a s_{t-1} + (1 - a) u_t`` (fp32) for u ``[B, T, N]``, a ``[N]``, s0 ``[B, N]`` or None.
    ``spin_limit`` bounds each tile's wait for its predecessors (``lng_ssm_scan_bounded``; None: the
    library's bound); a tile whose wait runs out forms its carry from u directly (exact).
    ``want_bf16``: returns ``(s, s rounded to bf16)`` from the same launch (``lng_ssm_scan_with_bf16``)."""
    dev = _dev(a, u, s0)
    uc = _c(u.float())
    ac = _c(a.float())
    s0c = None if s0 is None else _c(s0.float())
    b, t, n = uc.shape
    out = torch.empty_like(uc)
    ws = _ssm_workspace(dev, lib().lng_ssm_workspace_bytes(b, t, n))
    sb = None
    if want_bf16:
        if spin_limit is not None:
            raise ValueError("want_bf16 takes the library's wait bound")
        sb = torch.empty(b, t, n, dtype=torch.bfloat16, device=dev)
        launch = lambda: lib().lng_ssm_scan_with_bf16(_ptr(ac), _ptr(uc), _ptr(s0c), b, t, n, _ptr(ws),  # noqa: E731
                                                      ws.numel(), _ptr(out), _ptr(sb), _stream(dev))
    elif spin_limit is None:
        launch = lambda: lib().lng_ssm_scan(_ptr(ac), _ptr(uc), _ptr(s0c), b, t, n, _ptr(ws), ws.numel(),  # noqa: E731
                                            _ptr(out), _stream(dev))
    else:
        launch = lambda: lib().lng_ssm_scan_bounded(_ptr(ac), _ptr(uc), _ptr(s0c), b, t, n, _ptr(ws),  # noqa: E731
                                                    ws.numel(), int(spin_limit), _ptr(out), _stream(dev))
    check(_timed("ssm_scan", dev, launch), "ssm_scan")
    return (out, sb) if want_bf16 else out


def ssm_tree(a: torch.Tensor, u: torch.Tensor, parent, s_root: torch.Tensor | None = None) -> torch.Tensor:
    """States of a draft tree's nodes (``lng_ssm_tree``): node ``i`` continues from its parent's state,
    the root (parent -1) from ``s_root [B, N]`` or zero; u ``[B, n, N]`` -> s ``[B, n, N]`` fp32.
    ``parent``: a sequence or an int32 device tensor."""
    dev = _dev(a, u, s_root)
    uc = _c(u.float())
    ac = _c(a.float())
    b, n, nch = uc.shape
    par = parent.to(device=dev, dtype=torch.int32) if isinstance(parent, torch.Tensor) else \
        torch.as_tensor(list(parent), dtype=torch.int32).to(dev)
    if par.numel() != n:
        raise ValueError(f"ssm_tree: {par.numel()} parents for {n} nodes")
    sr = None if s_root is None else _c(s_root.float().reshape(b, nch))
    out = torch.empty_like(uc)
    check(lib().lng_ssm_tree(_ptr(ac), _ptr(uc), _ptr(sr), _ptr(par), b, n, nch, _ptr(out), _stream(dev)), "ssm_tree")
    return out


def ssm_scan_status(dev: torch.device) -> int:
    """Read and clear the status word of the current stream's scan workspace (bit 0: some tile of a
    call since the last read formed its carry directly, after its wait ran out).  Synchronises."""
    key = (dev.index, torch.cuda.current_stream(dev).cuda_stream)
    with _ssm_ws_lock:
        ws = _ssm_ws.get(key)
    if ws is None:
        return 0
    word = ws[:4].view(torch.int32)
    v = int(word.item())
    word.zero_()
    return v


def tree_accept(parent: torch.Tensor, node_tokens: torch.Tensor, argmax: torch.Tensor, out=None):
    """Device tree acceptance -> ``(path int32 [n], path_len int32 [1], new_tokens int64 [n])``
    (valid entries: the first ``path_len``).  ``out`` = (path, path_len, new_tokens) writes into
    caller tensors of those dtypes and sizes (e.g. views of one buffer, so that one copy brings
    the whole result to the host)."""
    dev = _dev(parent, node_tokens, argmax)
    n = parent.numel()
    p = _c(parent.to(torch.int32))
    nt = _c(node_tokens.to(torch.int64))
    am = _c(argmax.to(torch.int64))
    if out is None:
        path = torch.empty(n, dtype=torch.int32, device=dev)
        plen = torch.empty(1, dtype=torch.int32, device=dev)
        new = torch.empty(n, dtype=torch.int64, device=dev)
    else:
        path, plen, new = out
        if (path.dtype, plen.dtype, new.dtype) != (torch.int32, torch.int32, torch.int64) or \
                path.numel() < n or plen.numel() < 1 or new.numel() < n or \
                not all(x.is_contiguous() and x.device == p.device for x in (path, plen, new)):
            raise ValueError("tree_accept out: contiguous int32 [n], int32 [1], int64 [n] on the device")
    check(lib().lng_tree_accept(_ptr(p), _ptr(nt), _ptr(am), n, _ptr(path), _ptr(plen), _ptr(new), _stream(dev)),
          "tree_accept")
    return path, plen, new


def sink_logit_for(routes: int, mass: float = 0.5) -> float:
    return math.log(routes * (1.0 - mass) / mass)
