"""The allocation-free GQA decode entry point against the workspace entry point (GPU).

``flux_gqa_decode_attention_noalloc_f32`` runs the same kernels as
``flux_gqa_decode_attention_f32`` with the split-K partials in the library's
per-device scratch array, so its output must be bit-identical.  Two calls in a row,
the second smaller, show that the scratch the first call left behind does not leak
into the second; capacities beyond the scratch's maximum are refused.  Also checked
against the float64 oracle at the reference's tolerance (test_decode_ops.cu:158-250).
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from flux_amd import _native
from oracle import kernels as ref

pytestmark = pytest.mark.gpu

D = 64


def _inputs(device, capacity, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(9, D, generator=g).to(device)
    kc = torch.randn(3, capacity, D, generator=g).to(device)
    vc = torch.randn(3, capacity, D, generator=g).to(device)
    return q, kc, vc


def _with_workspace(lib, device, q, kc, vc, capacity, pos):
    ws_bytes = ctypes.c_int64()
    _native.check(lib.flux_gqa_decode_workspace_bytes(capacity, ctypes.byref(ws_bytes)))
    ws = torch.empty(ws_bytes.value // 4, device=device)
    out = torch.full((9, D), float("nan"), device=device)
    _native.check(lib.flux_gqa_decode_attention_f32(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), pos.data_ptr(),
                                                    capacity, 0.125, ws.data_ptr(), ws_bytes.value, out.data_ptr(),
                                                    _native.current_stream(device)))
    return out


def _no_alloc(lib, device, q, kc, vc, capacity, pos):
    out = torch.full((9, D), float("nan"), device=device)
    _native.check(lib.flux_gqa_decode_attention_noalloc_f32(q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                                            pos.data_ptr(), capacity, 0.125, out.data_ptr(),
                                                            _native.current_stream(device)))
    return out


def test_no_alloc_gqa_decode_matches_workspace_entry(gpu_device):
    lib = _native.load()
    # Largest capacity first (every one of the 85 chunks of partials in use), then a smaller call.
    for capacity, length, seed in ((16384, 16384, 71), (8704, 8193, 72), (300, 37, 73)):
        q, kc, vc = _inputs(gpu_device, capacity, seed)
        pos = torch.tensor([length - 1], dtype=torch.long, device=gpu_device)
        expected = _with_workspace(lib, gpu_device, q, kc, vc, capacity, pos)
        got = _no_alloc(lib, gpu_device, q, kc, vc, capacity, pos)
        torch.cuda.synchronize()
        assert torch.equal(got, expected), f"capacity {capacity}, length {length}"
        oracle = ref.gqa_decode_attention(q.cpu(), kc.cpu(), vc.cpu(), length, 0.125)
        torch.testing.assert_close(got.cpu().double(), oracle, rtol=3e-4, atol=3e-5)


def test_no_alloc_gqa_decode_refuses_capacity_beyond_scratch(gpu_device):
    lib = _native.load()
    q, kc, vc = _inputs(gpu_device, 8, 74)
    pos = torch.tensor([3], dtype=torch.long, device=gpu_device)
    out = torch.empty(9, D, device=gpu_device)
    status = lib.flux_gqa_decode_attention_noalloc_f32(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), pos.data_ptr(),
                                                       16385, 0.125, out.data_ptr(), _native.current_stream(gpu_device))
    assert status == 1  # FLUX_ERROR_INVALID_VALUE, before any launch
    assert b"16384" in lib.flux_last_error()
