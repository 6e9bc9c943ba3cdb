"""Seeded inputs and parameters shared by the golden-fixture generator and the tests that read
the fixtures (test infrastructure only).

Every array is drawn from numpy's legacy ``RandomState``, whose streams are fixed across numpy
versions, with a seed derived from the array's name.  A fixture therefore stores only the
outputs that the reference computed (plus small integer inputs); the tests rebuild the
floating-point inputs and parameters here and hand them to the oracle.

Parameter rules (by state-dict key or bundle array name):

- norm weights (``*norm*``) and the SSM decay are drawn around their natural values
  (``1 + 0.1 N(0,1)`` and ``U[0.6, 0.99]``), so a swapped or dropped weight shows;
- the short-conv weight is ``N(0, 0.2)``; every other weight, table and the start vector is
  ``N(0, 0.02)``, drawn in fp32 and cast afterwards, like the reference's ``_normal_init``.
"""

from __future__ import annotations

import zlib

import numpy as np


def _seed(name: str, base: int) -> int:
    return (zlib.crc32(name.encode()) ^ (base * 0x9E3779B1)) & 0x7FFFFFFF


def normal(name: str, shape, std: float = 1.0, mean: float = 0.0, base: int = 0) -> np.ndarray:
    rs = np.random.RandomState(_seed(name, base))
    return (mean + std * rs.standard_normal(tuple(shape))).astype(np.float32)


def uniform(name: str, shape, lo: float, hi: float, base: int = 0) -> np.ndarray:
    rs = np.random.RandomState(_seed(name, base))
    return rs.uniform(lo, hi, tuple(shape)).astype(np.float32)


def integers(name: str, shape, lo: int, hi: int, base: int = 0) -> np.ndarray:
    rs = np.random.RandomState(_seed(name, base))
    return rs.randint(lo, hi, tuple(shape)).astype(np.int64)


def param(name: str, shape, base: int = 0) -> np.ndarray:
    """One parameter by the rules above (fp32)."""
    if "norm" in name:
        return normal(name, shape, 0.1, 1.0, base)
    if "conv.weight" in name:
        return normal(name, shape, 0.2, 0.0, base)
    if name in ("ssm_decay",):
        return uniform(name, shape, 0.6, 0.99, base)
    return normal(name, shape, 0.02, 0.0, base)


def state(shapes: dict, base: int = 0) -> dict:
    """A state dict ``{key: fp32 array}`` for ``{key: shape}``."""
    return {k: param(k, s, base) for k, s in shapes.items()}


# ------------------------------------------------------------------ configurations
# Tiny fp32 memory layer: the C1 widths (d 128, 8 routes, mem_dim 32, 4 query heads x 32, 2 KV heads).
TINY_MEM = dict(d_model=128, cfg=dict(routes=8, mem_dim=32, head_dim=32, q_heads=4, kv_heads=2))
# bf16 memory layer at the SB widths (d 1024, mem_dim 128, 16 query heads x 64, 4 KV heads), 32 routes.
SB_MEM = dict(d_model=1024, cfg=dict(routes=32, mem_dim=128, head_dim=64, q_heads=16, kv_heads=4))

# Tiny drafter bundles (bundle_config keys of drafting/export_drafter.py:212-215).
_DRAFT_BASE = dict(d_model=64, vocab=96, routes=4, bits=4, ngrams=[2, 3], mem_dim=16, kv_heads=2, head_dim=16,
                   q_heads=4, norm_eps=1e-5, ssm_eps=1e-5, router_eps=1e-5, draft_eps=1e-5, mem_eps=1e-5,
                   softmax_scale=0.25, sink_logit=float(np.log(4.0)), table_dtype="fp16", layer=1)


def drafter_config(kind: str, sketch_k: int = 0, cap: int = 0) -> dict:
    """``sdb`` (embed2 router, no SSM) or ``sdc`` (embed2_ssm router, SSM state in the query)."""
    c = dict(_DRAFT_BASE)
    if kind == "sdb":
        c.update(kind="sd_b", router_kind="embed2", ssm_dim=0, query_ssm=False)
    elif kind == "sdc":
        c.update(kind="sd_c", router_kind="embed2_ssm", ssm_dim=8, query_ssm=True)
    else:
        raise ValueError(kind)
    c.update(sketch_k=sketch_k, shortlist_cap=cap if sketch_k else 0)
    c["groups"] = c["q_heads"] // c["kv_heads"]
    c["route_token_dim"] = len(c["ngrams"]) * c["mem_dim"]
    return c


def drafter_arrays(cfg: dict, base: int = 0) -> dict:
    """Bundle arrays (``export_drafter.py:15-33`` layout) for ``cfg``: fp32 weights, fp16 tables,
    uint16 / uint32 sketches and an int32 fallback list when ``sketch_k > 0``."""
    d, V, R, md = cfg["d_model"], cfg["vocab"], cfg["routes"], cfg["mem_dim"]
    kh, inner, dt = cfg["kv_heads"] * cfg["head_dim"], cfg["q_heads"] * cfg["head_dim"], cfg["route_token_dim"]
    n_state = cfg["ssm_dim"]
    feat = 2 * d + (n_state if cfg["router_kind"] == "embed2_ssm" else 0)
    shapes = {"embedding": (V, d), "mem_norm": (dt,), "kv_proj": (2 * kh, dt), "router": (R * cfg["bits"], feat),
              "router_prev_norm": (d,), "router_cur_norm": (d,), "router_start": (d,), "q_norm": (d,),
              "w_q": (inner, d), "w_o": (d, inner), "out_norm": (d,)}
    if n_state:
        shapes.update(ssm_norm=(d,), ssm_w_in=(n_state, d), ssm_decay=(n_state,))
    if cfg["query_ssm"]:
        shapes["w_sq"] = (inner, n_state)
    out = state(shapes, base)
    # the embedding is the draft query input and the unembedding: unit scale keeps logits O(1)
    out["embedding"] = normal("embedding", (V, d), 1.0, 0.0, base)
    for n in cfg["ngrams"]:
        rows = R * (1 << (cfg["bits"] * n))
        out[f"table_{n}"] = normal(f"table_{n}", (rows, md), 0.02, 0.0, base).astype(np.float16)
    k = int(cfg.get("sketch_k", 0))
    if k:
        for n in cfg["ngrams"]:
            rows = R * (1 << (cfg["bits"] * n))
            out[f"sketch_ids_{n}"] = integers(f"sketch_ids_{n}", (rows, k), 0, V, base).astype(np.uint16)
            cnt = integers(f"sketch_counts_{n}", (rows, k), 0, 4, base)
            out[f"sketch_counts_{n}"] = cnt.astype(np.uint32)   # count 0 = empty slot
        out["fallback"] = integers("fallback", (12,), 0, V, base).astype(np.int32)
    return out


# ------------------------------------------------------------------ lookup surrogate (training)
# (name, order, bits, routes, route_start, batch, time, mem_dim, dtype, temperature, scale, exact)
SURROGATE_CASES = [
    ("sg_o2_f32_approx", 2, 4, 3, 1, 2, 7, 32, "f32", 0.7, 1.3, False),
    ("sg_o2_f32_exact", 2, 4, 3, 1, 2, 7, 32, "f32", 0.7, 1.3, True),
    ("sg_o3_bf16_approx", 3, 4, 2, 0, 2, 9, 32, "bf16", 1.0, 1.0, False),
    ("sg_o3_bf16_exact", 3, 4, 2, 0, 2, 9, 32, "bf16", 1.0, 1.0, True),
    ("sg_o3_b2_f32_approx", 3, 2, 4, 2, 1, 11, 64, "f32", 1.5, 0.5, False),
    ("sg_o3_b2_f32_exact", 3, 2, 4, 2, 1, 11, 64, "f32", 1.5, 0.5, True),
]


def surrogate_inputs(case) -> dict:
    """Inputs of one surrogate case: the order's table (rows for routes 0 .. route_start + R - 1),
    codes of the R routes, route logits, the memory gradient and the valid tokens (one position of
    the first sequence invalid).  All fp32 / int64; the case's dtype is applied by the user."""
    name, order, bits, R, rs, B, T, D = case[:8]
    A = 1 << bits
    rows = (rs + R) * A ** order
    valid = np.ones((B, T), dtype=bool)
    valid[0, min(T - 1, order + 1)] = False
    return {"table": normal(f"{name}_table", (rows, D)),
            "codes": integers(f"{name}_codes", (B, T, R), 0, A),
            "q": normal(f"{name}_q", (B, T, R, bits)),
            "grad": normal(f"{name}_grad", (B, T, R, D)),
            "valid_tokens": valid}


# ------------------------------------------------------------------ online counts (drafting)
# (name, time, routes, vocab, orders, kappa)
ONLINE_CASES = [
    ("oc_o23_k1", 48, 4, 20, (2, 3), 1.0),
    ("oc_o23_k05", 48, 4, 20, (2, 3), 0.5),
    ("oc_o3_k1", 40, 3, 12, (3,), 1.0),
    ("oc_o2_r1_k05", 36, 1, 9, (2,), 0.5),
]


def online_inputs(case) -> dict:
    """Inputs of one online-count case (``OnlineCounts(codes, x, orders, 4, V, kappa).mix``).

    The committed codes ``[T, R]`` use the values 0..11: their first half is random, the second
    half repeats a 4-step pattern, so windows taken there match many earlier pairs.  Eight query
    windows ``[8, 3, R]`` with their real masks and deadlines:

    0. a window of the repeating half (many matches, every pair verified);
    1. the same window with a deadline that cuts the later matches;
    2. a window of the random half (at least its own pair matches);
    3. codes 12..15 only, which no committed code has (no match);
    4. window 0 with its oldest position before the sequence start (order 3 invalid, order 2 counts);
    5. only the newest position real (no order is valid: the distribution is unchanged);
    6. window 0 with nothing verified yet (deadline -1);
    7. window 2's newest two codes after a changed oldest code (order 2 matches, order 3 not).

    ``p`` is a softmax of random logits (fp32)."""
    name, T, R, V = case[:4]
    half = T // 2
    codes = integers(f"{name}_codes", (T, R), 0, 12)
    pat = integers(f"{name}_pat", (4, R), 0, 12)
    codes[half:] = pat[np.arange(T - half) % 4]
    x = integers(f"{name}_x", (T,), 0, V)
    ta, tb = T - 6, half - 5                  # window ends: repeating half, random half
    w0, w2 = codes[ta - 2: ta + 1], codes[tb - 2: tb + 1]
    w7 = w2.copy()
    w7[0] = (w7[0] + 1) % 12
    win = np.stack([w0, w0, w2, integers(f"{name}_none", (3, R), 12, 16), w0, w0, w0, w7])
    real = np.ones((8, 3), dtype=bool)
    real[4, 0] = False
    real[5, :2] = False
    deadline = np.array([T - 2, half + 6, T - 2, T - 2, T - 2, T - 2, -1, T - 2], dtype=np.int64)
    logits = normal(f"{name}_logits", (8, V))
    p = np.exp(logits - logits.max(1, keepdims=True))
    p = (p / p.sum(1, keepdims=True)).astype(np.float32)
    return {"codes": codes, "x": x, "win": win, "real": real, "deadline": deadline, "p": p}
