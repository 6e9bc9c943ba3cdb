"""The allocation-free scan entry point ``lng_ssm_scan_static`` against ``lng_ssm_scan`` (GPU), both
called through the C ABI: bit-identical states on two calls in a row, the second one smaller; replays
of a HIP graph that captured it, with new inputs each time; and the refusal of a shape past its static
scratch (which launches nothing)."""

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
                                ws.data_ptr(), nbytes, out.data_ptr(), st), "ssm_scan")
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


def test_static_scan_replayed_from_a_graph(dev):
    # the epoch that tags the hand-off records lives in the static array, so every replay of one
    # captured launch accepts only its own records: each replay, with new inputs copied in between
    # (and eager work of the program in between), equals the workspace scan of those inputs
    lib = _lib.load()
    g = torch.Generator().manual_seed(9)
    b, t, n = 8, 4096, 256
    a = (0.9 + 0.099 * torch.rand(n, generator=g)).to(dev)
    u = torch.empty(b, t, n, device=dev)
    out = torch.empty_like(u)
    u.copy_(torch.randn(b, t, n, generator=g).to(dev))
    _scan_static(lib, a, u, None)          # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        st = torch.cuda.current_stream(dev).cuda_stream
        _lib.check(lib.lng_ssm_scan_static(a.data_ptr(), u.data_ptr(), 0, b, t, n, out.data_ptr(), st),
                   "ssm_scan_static")
    for rep in range(4):
        u.copy_(torch.randn(b, t, n, generator=g).to(dev))
        _scan_with_workspace(lib, a, u.flip(1).contiguous(), None)    # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = _scan_with_workspace(lib, a, u, None)
        torch.cuda.synchronize()
        assert torch.equal(out, want), rep
    status = torch.zeros(1, dtype=torch.int32)
    _lib.check(lib.lng_ssm_scan_static_status(status.data_ptr()), "ssm_scan_static_status")
    assert int(status) == 0
