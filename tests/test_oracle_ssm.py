"""Oracle pinning for the diagonal SSM scan (CPU).

``ssm_scan`` (the sequential recurrence, ``ssm.py:58-65``) is checked against the
closed form for a constant input, against a chunked restatement built like the
reference's ``chunked_scan`` (``ssm.py:68-91``: a^(t-k) decay matrix inside chunks,
a^(t+1) carry across chunks), and the carried-state form (``infer.py:125-137``).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import memory as om


def chunked_restatement(a, u, chunk):
    b, t, n = u.shape
    L = min(chunk, t)
    pad = (-t) % L
    x = np.pad((1 - a) * u, ((0, 0), (0, pad), (0, 0)))
    c = x.shape[1] // L
    idx = np.arange(L)
    diff = idx[:, None] - idx[None, :]
    decay = np.where(diff[..., None] >= 0, a[None, None, :] ** np.maximum(diff, 0)[..., None], 0.0)  # [L, L, N]
    out = np.zeros((b, c * L, n))
    state = np.zeros((b, n))
    carry = a[None, :] ** (idx[:, None] + 1)  # [L, N]
    for ci in range(c):
        xs = x[:, ci * L:(ci + 1) * L]
        local = np.einsum("tkn,bkn->btn", decay, xs)
        blk = local + carry[None] * state[:, None]
        out[:, ci * L:(ci + 1) * L] = blk
        state = blk[:, -1]
    return out[:, :t]


def test_constant_input_closed_form():
    rng = np.random.default_rng(0)
    a = rng.uniform(0.5, 0.999, 16)
    u = rng.standard_normal(16)
    s0 = rng.standard_normal((1, 16))
    t = 300
    got = om.ssm_scan(a, np.broadcast_to(u, (1, t, 16)), s0)
    want = om.ssm_scan_closed_form_constant(a, u, t, s0[0])
    np.testing.assert_allclose(got[0], want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("t,chunk", [(2048, 128), (301, 64), (5, 8)])
def test_sequential_equals_chunked(t, chunk):
    rng = np.random.default_rng(t)
    a = rng.uniform(0.9, 0.999, 12)
    u = rng.standard_normal((2, t, 12))
    np.testing.assert_allclose(om.ssm_scan(a, u), chunked_restatement(a, u, chunk), rtol=1e-9, atol=1e-9)


def test_carried_state_equals_continuation():
    rng = np.random.default_rng(3)
    a = rng.uniform(0.5, 0.999, 8)
    u = rng.standard_normal((3, 40, 8))
    full = om.ssm_scan(a, u)
    tail = om.ssm_scan(a, u[:, 25:], full[:, 24])
    np.testing.assert_allclose(tail, full[:, 25:], rtol=1e-12, atol=1e-12)
