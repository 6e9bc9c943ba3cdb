"""Oracle pinning for the integer parts: codes, n-gram addresses, rows (CPU).

Known-answer tests are the reference's own (``tests/test_index_layout.py:28-45``,
``docs/VERIFIED.md:7-28``); the Python and C restatements are cross-checked on random
inputs and against brute force over explicit windows.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import cint
from oracle import memory as om


def test_digit_order_known_answers():
    # reference tests/test_index_layout.py:28-33 -- one route, codes 3,5,7,9
    codes = np.array([[[3], [5], [7], [9]]])
    a2 = om.ngram_address(codes, 2, 4)
    a3 = om.ngram_address(codes, 3, 4)
    assert a2[0, 0, 0] == 3 + 16 * 5          # window (c0=3, c1=5): oldest least significant
    assert a3[0, 1, 0] == 5 + 16 * 7 + 256 * 9  # window ending at t = 3
    assert a2.shape == (1, 3, 1) and a3.shape == (1, 2, 1)


def test_rows_layout_known_answers():
    # docs/VERIFIED.md:14-16: 2-gram row = r*256 + c[t-1] + 16 c[t]; 3-gram = r*4096 + c[t-2] + 16 c[t-1] + 256 c[t]
    rng = np.random.default_rng(0)
    codes = rng.integers(0, 16, (2, 7, 5))
    rows = om.route_rows(codes, (2, 3), 4)
    for b in range(2):
        for t in range(7):
            for r in range(5):
                want2 = r * 256 + codes[b, t - 1, r] + 16 * codes[b, t, r] if t >= 1 else -1
                want3 = (r * 4096 + codes[b, t - 2, r] + 16 * codes[b, t - 1, r] + 256 * codes[b, t, r]
                         if t >= 2 else -1)
                assert rows[b, t, r, 0] == want2 and rows[b, t, r, 1] == want3


def test_zero_rows_before_order_minus_one():
    # tests/test_index_layout.py:34-39: nothing complete at t = 0, no 3-gram at t = 1
    rng = np.random.default_rng(1)
    codes = rng.integers(0, 16, (1, 6, 4))
    import torch

    tables = {2: torch.randn(4 * 256, 8), 3: torch.randn(4 * 4096, 8)}
    tok = om.route_tokens(tables, codes, (2, 3), 4)
    assert torch.count_nonzero(tok[:, 0]) == 0
    assert torch.count_nonzero(tok[:, 1, :, 8:]) == 0
    assert torch.count_nonzero(tok[:, 1, :, :8]) > 0


def test_pack_codes_strict_sign_rule():
    # lngram_v2.py:1017 -- bit = (q > 0): 0, -0 and NaN give 0
    q = np.array([[0.0, -0.0, np.nan, 1e-30, -1e-30, 5.0, -5.0, 0.0]], np.float32)
    codes = om.pack_route_codes(q, 4)
    assert codes.tolist() == [[0b1000, 0b0010]]
    assert cint.pack_codes(q, 4).tolist() == codes.tolist()


def test_pack_codes_bit_order_and_c_restatement():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((33, 4 * 9)).astype(np.float32)
    codes = om.pack_route_codes(q, 4)
    brute = np.zeros_like(codes)
    for m in range(33):
        for r in range(9):
            brute[m, r] = sum(int(q[m, 4 * r + i] > 0) << i for i in range(4))
    np.testing.assert_array_equal(codes, brute)
    np.testing.assert_array_equal(cint.pack_codes(q, 4), codes)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_rows_c_equals_python_with_segments_and_valid(seed):
    rng = np.random.default_rng(seed)
    b, t, r = 3, 11, 6
    codes = rng.integers(0, 16, (b, t, r))
    seg = np.cumsum(rng.random((b, t)) < 0.2, axis=1).astype(np.int32)
    valid = rng.random((b, t)) < 0.8
    for s, v in ((None, None), (seg, None), (None, valid), (seg, valid)):
        py = om.route_rows(codes, (2, 3), 4, segment_ids=s, valid_tokens=v)
        c = cint.ngram_rows(codes, (2, 3), 4, s, v)
        np.testing.assert_array_equal(py, c)


def test_segment_rule_compares_window_ends():
    # _valid_mask (lngram_v2.py:1027-1045) compares the first and the last position of the window
    codes = np.zeros((1, 4, 1), np.int64)
    seg = np.array([[0, 1, 1, 1]])
    rows = om.route_rows(codes, (2, 3), 4, segment_ids=seg)
    assert rows[0, :, 0, 0].tolist() == [-1, -1, 0, 0]      # 2-gram windows (0,1) cross, (1,2), (2,3) ok
    assert rows[0, :, 0, 1].tolist() == [-1, -1, -1, 0]     # 3-gram windows (0..2) cross, (1..3) ok


def test_route_chunk_offsets_use_absolute_route():
    # lngram_v2.py:1070-1077: offsets = arange(route_start, route_end) * 16^n
    codes = np.full((1, 3, 8), 1)
    rows = om.route_rows(codes, (2,), 4, route_start=5, route_end=8)
    assert rows.shape == (1, 3, 3, 1)
    assert rows[0, 2, :, 0].tolist() == [5 * 256 + 17, 6 * 256 + 17, 7 * 256 + 17]
