"""The allocation-free scan entry point ``lng_ssm_scan_static`` against ``lng_ssm_scan`` (GPU), both
called through the C ABI: bit-identical states on two calls in a row, the second one smaller, and
the refusal of a shape past its static scratch (which launches nothing)."""

from __future__ import annotations

import pytest
import torch

from lngram_hip import _lib, ops

pytestmark = pytest.mark.gpu


def _scan_with_workspace(lib, a, u, s0):
    b, t, n = u.shape
    nbytes = lib.lng_ssm_workspace_bytes(b, t, n)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=u.device)
    out = torch.empty_like(u)
    st = torch.cuda.current_stream(u.device).cuda_stream
    _lib.check(lib.lng_ssm_scan(a.data_ptr(), u.data_ptr(), 0 if s0 is None else s0.data_ptr(), b, t, n,
                                ws.data_ptr(), nbytes, 7, out.data_ptr(), st), "ssm_scan")
    return out


def _scan_static(lib, a, u, s0):
    b, t, n = u.shape
    out = torch.empty_like(u)
    st = torch.cuda.current_stream(u.device).cuda_stream
    _lib.check(lib.lng_ssm_scan_static(a.data_ptr(), u.data_ptr(), 0 if s0 is None else s0.data_ptr(), b, t, n,
                                       out.data_ptr(), st), "ssm_scan_static")
    return out


def test_static_scan_matches_workspace_scan(dev):
    lib = _lib.load()
    g = torch.Generator().manual_seed(3)
    for b, t, n, with_s0 in ((8, 4096, 256, False), (3, 301, 70, True)):
        a = (0.9 + 0.099 * torch.rand(n, generator=g)).to(dev)
        u = torch.randn(b, t, n, generator=g).to(dev)
        s0 = torch.randn(b, n, generator=g).to(dev) if with_s0 else None
        got = _scan_static(lib, a, u, s0)
        want = _scan_with_workspace(lib, a, u, s0)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (b, t, n)
    # past the static scratch: refused with a clear error before any launch
    b, t, n = 17, 16384, 256   # 17 * 128 tiles > 2048
    rc = lib.lng_ssm_scan_static(0, 0, 0, b, t, n, 0, 0)
    assert rc == -1 and b"2048 tiles" in lib.lng_last_error()
