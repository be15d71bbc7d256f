"""C-ABI boundary checks that need no GPU: the library loads, exports exactly what
include/flux_amd.h declares, and rejects invalid arguments before any launch
(reference launchers return cudaErrorInvalidValue the same way, e.g.
csrc/packed_gate_up_gemv/packed_gate_up_gemv_cuda.cu:57-59)."""

from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

from flux_amd import _native
from tests.conftest import ROOT

HEADER = os.path.join(ROOT, "include", "flux_amd.h")


def _declared_functions() -> set[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(flux_[a-z0-9_]+)\s*\(", text))


def test_library_exports_every_declared_symbol():
    lib = _native.load()
    declared = _declared_functions()
    assert len(declared) >= 30
    for name in sorted(declared):
        assert hasattr(lib, name), f"{name} declared in include/flux_amd.h but not exported"
    assert declared == set(_native.EXPORTED_SYMBOLS), "ctypes prototypes and header disagree"


def test_exported_symbols_match_nm():
    out = subprocess.run(["nm", "-D", "--defined-only", _native.LIBRARY_PATH], capture_output=True, text=True)
    if out.returncode != 0:
        pytest.skip("nm unavailable")
    exported = {line.split()[-1] for line in out.stdout.splitlines() if " T flux_" in line}
    assert _declared_functions() <= exported


def test_version_and_empty_error():
    lib = _native.load()
    assert b"gfx950" in lib.flux_version()


@pytest.mark.parametrize("call", [
    lambda lib: lib.flux_rmsnorm_f32(None, None, None, 1, 576, 1e-5, None),
    lambda lib: lib.flux_residual_rmsnorm_f32(None, None, None, None, None, 1, 576, 1e-5, None),
    lambda lib: lib.flux_qkv_rope_cache_f32(None, None, 1e-5, None, None, None, None, 8, None, None, None, None),
    lambda lib: lib.flux_gqa_decode_attention_f32(None, None, None, None, 8, 0.125, None, 0, None, None),
    lambda lib: lib.flux_linear576_f32(None, None, None, None, 576, None),
    lambda lib: lib.flux_gate_up_swiglu_f32(None, None, 0.0, None, None, None),
    lambda lib: lib.flux_down_residual_f32(None, None, None, None, None),
    lambda lib: lib.flux_greedy_argmax_f32(None, 10, None, None),
    lambda lib: lib.flux_greedy_argmax_update_f32(None, 10, None, None, None, 4, None, None, None),
    lambda lib: lib.flux_linear_f32(None, None, None, None, 4, 64, 16, None),
    lambda lib: lib.flux_gate_up_swiglu_rows_f32(None, None, None, 4, None),
    lambda lib: lib.flux_qkv_rope_cache_rows_f32(None, None, None, None, 4, None, None, None, 8, None),
    lambda lib: lib.flux_prefill_attention_f32(None, None, None, 4, 8, 0.125, None, None, None),
    lambda lib: lib.flux_embedding_gather_f32(None, None, 10, 4, None, None),
    lambda lib: lib.flux_decode_create(None, None, None, 8, 0, None, None, None, None, None, None, None, None),
    lambda lib: lib.flux_prefill_create(None, None, None, 8, None, 4, None, None, None, None),
    lambda lib: lib.flux_decode_replay(None, None, None, None),
    lambda lib: lib.flux_decode_generate_greedy(None, 1, None, None),
    lambda lib: lib.flux_prefill_run(None, None, None, None),
])
def test_null_arguments_are_rejected_without_a_launch(call):
    lib = _native.load()
    assert call(lib) == _native.FLUX_ERROR_INVALID_VALUE
    assert _native.last_error()


def test_shape_constraints_are_rejected():
    lib = _native.load()
    dummy = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    assert lib.flux_linear_f32(dummy, dummy, None, dummy, 4, 60, 16, None) == _native.FLUX_ERROR_INVALID_VALUE
    assert lib.flux_linear_f32(dummy, dummy, None, dummy, 4, 64, 10, None) == _native.FLUX_ERROR_INVALID_VALUE
    assert "n % 64" in _native.last_error()
    size = ctypes.c_int64()
    assert lib.flux_gqa_decode_workspace_bytes(16385, ctypes.byref(size)) == _native.FLUX_ERROR_INVALID_VALUE
    assert lib.flux_gqa_decode_workspace_bytes(8192, ctypes.byref(size)) == _native.FLUX_OK
    assert size.value == 85 * 3 * 3 * 66 * 4
    # Keys are split into chunks of 2 to 24 64-key tiles (longer for longer prompts): a single
    # 128-query tile never needs partials.
    assert lib.flux_prefill_attention_workspace_bytes(128, ctypes.byref(size)) == _native.FLUX_OK
    assert size.value == 0
    # 2048 tokens: 4-tile chunks; the 14 query tiles past the first 2 x 9 heads x 8 chunks
    # x 128 rows x (64 + m + l + 2 pad) floats
    assert lib.flux_prefill_attention_workspace_bytes(2048, ctypes.byref(size)) == _native.FLUX_OK
    assert size.value == 14 * 9 * 8 * 128 * 68 * 4
    # 8192 tokens: 16-tile (1024-key) chunks, 56 query tiles past the first 8, 8 chunks
    assert lib.flux_prefill_attention_workspace_bytes(8192, ctypes.byref(size)) == _native.FLUX_OK
    assert size.value == 56 * 9 * 8 * 128 * 68 * 4
    dummy = ctypes.c_void_p(16)
    assert lib.flux_prefill_attention_f32(dummy, dummy, dummy, 4096, 4096, 0.125, None, dummy,
                                          None) == _native.FLUX_ERROR_INVALID_VALUE
    assert "workspace" in _native.last_error()
    assert lib.flux_prefill_attention_f32(dummy, dummy, dummy, 64, 64, 0.125, None, ctypes.c_void_p(20),
                                          None) == _native.FLUX_ERROR_INVALID_VALUE
    assert "16-byte aligned" in _native.last_error()


def test_runtime_constructor_validation_messages():
    lib = _native.load()
    weights = _native.FluxWeights()  # all null pointers
    weights.vocab_size = 0
    handle = ctypes.c_void_p()
    eps = _native.double_array([1e-5] * 30)
    scale = _native.double_array([0.125] * 30)
    status = lib.flux_decode_create(ctypes.byref(weights), None, None, 8, 0, None, None, None, None, eps, scale, None,
                                    ctypes.byref(handle))
    assert status == _native.FLUX_ERROR_INVALID_VALUE
    assert "vocabulary must be non-empty" in _native.last_error()
    weights.vocab_size = 128
    status = lib.flux_prefill_create(ctypes.byref(weights), None, None, 8, None, 4, eps, scale, None,
                                     ctypes.byref(handle))
    assert status == _native.FLUX_ERROR_INVALID_VALUE
    assert "required" in _native.last_error()
