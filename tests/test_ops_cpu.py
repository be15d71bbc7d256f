"""``torch.ops.flux`` contracts that need no GPU: registered schemas, argument
errors (same messages as the reference's TORCH_CHECKs), FakeTensor shapes, the
GPU-only contract of CPU tensors, and the missing-library error.

Mirrors the CPU-runnable parts of the reference's tests/test_ops.py:77-580.
"""

from __future__ import annotations

import math

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensor, FakeTensorMode

from flux_amd import _native, ops
from flux_amd.ops import native as native_ops

EPSILON = 1e-5

REFERENCE_SCHEMAS = {
    "rmsnorm": "flux::rmsnorm(Tensor input, Tensor weight, float epsilon) -> Tensor",
    "rmsnorm_out": "flux::rmsnorm_out(Tensor input, Tensor weight, float epsilon, Tensor(a!) output) -> Tensor(a!)",
    "residual_rmsnorm": ("flux::residual_rmsnorm(Tensor hidden, Tensor residual, Tensor weight, float epsilon) -> "
                         "(Tensor norm_out, Tensor residual_out)"),
    "residual_rmsnorm_out": ("flux::residual_rmsnorm_out(Tensor hidden, Tensor residual, Tensor weight, "
                             "float epsilon, Tensor(a!) norm_out, Tensor(b!) residual_out) -> "
                             "(Tensor(a!), Tensor(b!))"),
    "rope": "flux::rope(Tensor query, Tensor key, Tensor cos, Tensor sin) -> (Tensor, Tensor)",
    "softmax": "flux::softmax(Tensor input) -> Tensor",
    "attention_score_softmax": ("flux::attention_score_softmax(Tensor scores, Tensor additive_attention_mask, "
                                "float scale) -> Tensor"),
    "packed_swiglu": "flux::packed_swiglu(Tensor packed) -> Tensor",
    "packed_swiglu_out": "flux::packed_swiglu_out(Tensor packed, Tensor(a!) output) -> Tensor(a!)",
    "gqa_decode_attention": ("flux::gqa_decode_attention(Tensor query, Tensor key_cache, Tensor value_cache, "
                             "Tensor? additive_attention_mask, float scale, Tensor? cache_length=None) -> Tensor"),
    "gqa_decode_attention_out": ("flux::gqa_decode_attention_out(Tensor query, Tensor key_cache, "
                                 "Tensor value_cache, Tensor? additive_attention_mask, float scale, "
                                 "Tensor? cache_length, Tensor(a!) output, Tensor(b!) workspace) -> Tensor(a!)"),
    "packed_qkv_rope_cache": ("flux::packed_qkv_rope_cache(Tensor packed_qkv, Tensor cos, Tensor sin, "
                              "Tensor(a!) key_cache, Tensor(b!) value_cache, Tensor(c!) cache_length) -> Tensor"),
    "packed_qkv_rope_cache_out": ("flux::packed_qkv_rope_cache_out(Tensor packed_qkv, Tensor cos, Tensor sin, "
                                  "Tensor(a!) key_cache, Tensor(b!) value_cache, Tensor(c!) cache_length, "
                                  "Tensor(d!) query_output) -> Tensor(d!)"),
    "packed_gate_up_swiglu_out": ("flux::packed_gate_up_swiglu_out(Tensor input, Tensor weight, Tensor(a!) output)"
                                  " -> Tensor(a!)"),
}


def _wave(shape: tuple[int, ...]) -> torch.Tensor:
    values = torch.arange(math.prod(shape), dtype=torch.float32)
    return (torch.sin(values * 0.013) + torch.cos(values * 0.007)).reshape(shape)


def test_registered_schemas_match_the_reference():
    assert set(ops.OPERATOR_NAMES) == set(REFERENCE_SCHEMAS)
    for name, schema in REFERENCE_SCHEMAS.items():
        assert str(getattr(torch.ops.flux, name).default._schema) == schema, name


def test_availability_follows_the_native_library():
    available = _native.is_available()
    for probe in (ops.native_rmsnorm_is_available, ops.native_residual_rmsnorm_is_available,
                  ops.native_rope_is_available, ops.native_softmax_is_available,
                  ops.native_attention_score_softmax_is_available, ops.native_packed_swiglu_is_available,
                  ops.native_gqa_decode_attention_is_available, ops.native_packed_qkv_rope_cache_is_available,
                  ops.native_packed_gate_up_gemv_is_available):
        assert probe() == available
    assert (ops.native_rmsnorm_load_error() is None) == available


def test_missing_library_raises_not_built(monkeypatch):
    def missing(*_args, **_kwargs):
        raise RuntimeError("flux_amd native library is not built")

    monkeypatch.setattr(_native, "load", missing)
    assert not ops.native_rmsnorm_is_available()
    assert isinstance(ops.native_rmsnorm_load_error(), OSError)
    with pytest.raises(RuntimeError, match="Flux native RMSNorm is not built"):
        ops.rms_norm_native(torch.ones(2, 3), torch.ones(3), EPSILON)
    with pytest.raises(RuntimeError, match="not built"):
        ops.gqa_decode_attention_native(torch.ones(1, 9, 1, 64), torch.ones(1, 3, 4, 64), torch.ones(1, 3, 4, 64),
                                        None, 0.125)


@pytest.mark.parametrize("call", [
    lambda: ops.rms_norm_native(_wave((2, 7, 576)), torch.ones(576), EPSILON),
    lambda: ops.residual_rmsnorm_native(_wave((2, 576)), _wave((2, 576)), torch.ones(576), EPSILON),
    lambda: ops.softmax_native(_wave((5, 129))),
    lambda: ops.attention_score_softmax_native(_wave((2, 3, 5, 17)), _wave((2, 1, 5, 17)), 0.25),
    lambda: ops.packed_swiglu_native(_wave((1, 7, 3072))),
    lambda: ops.rope_native(_wave((1, 9, 3, 64)), _wave((1, 3, 3, 64)), _wave((1, 3, 64)), _wave((1, 3, 64))),
    lambda: ops.gqa_decode_attention_native(_wave((1, 9, 1, 64)), _wave((1, 3, 17, 64)), _wave((1, 3, 17, 64)),
                                            None, 0.125, torch.tensor(11)),
])
def test_cpu_tensors_are_rejected_after_validation(call):
    with pytest.raises(RuntimeError, match="no CPU kernel"):
        call()


def test_rmsnorm_error_contract():
    cases = (
        (torch.tensor(1.0), torch.ones(1), EPSILON, "at least one dimension"),
        (torch.ones(2, 3), torch.ones(2), EPSILON, "weight length"),
        (torch.ones(2, 3), torch.ones(3, dtype=torch.float64), EPSILON, "weight must have dtype torch.float32"),
        (torch.ones(2, 3), torch.ones(3), 0.0, "epsilon must be a positive"),
        (torch.ones(2, 3), torch.ones(3), float("nan"), "epsilon must be a positive"),
    )
    for input, weight, epsilon, message in cases:
        with pytest.raises(RuntimeError, match=message):
            ops.rms_norm_native(input, weight, epsilon)
    with pytest.raises(RuntimeError, match="inference-only"):
        ops.rms_norm_native(torch.ones(2, 3, requires_grad=True), torch.ones(3), EPSILON)
    with torch.no_grad(), pytest.raises(RuntimeError, match="no CPU kernel"):
        ops.rms_norm_native(torch.ones(2, 3, requires_grad=True), torch.ones(3), EPSILON)


def test_residual_rmsnorm_error_contract():
    cases = (
        (torch.ones(2, 3), torch.ones(1, 3), torch.ones(3), EPSILON, "same shape"),
        (torch.ones(2, 3), torch.ones(2, 3), torch.ones(2), EPSILON, "weight length"),
        (torch.ones(2, 3, dtype=torch.float64), torch.ones(2, 3), torch.ones(3), EPSILON,
         "hidden must have dtype torch.float32"),
        (torch.ones(2, 3), torch.ones(2, 3), torch.ones(3), float("inf"), "finite"),
        (torch.ones(2, 3), torch.ones(2, 3), torch.ones(3), -1.0, "non-negative"),
    )
    for hidden, residual, weight, epsilon, message in cases:
        with pytest.raises(RuntimeError, match=message):
            ops.residual_rmsnorm_native(hidden, residual, weight, epsilon)
    with pytest.raises(RuntimeError, match="inference-only"):
        ops.residual_rmsnorm_native(torch.ones(2, 3, requires_grad=True), torch.ones(2, 3), torch.ones(3), EPSILON)
    # epsilon == 0 is accepted (non-negative), as in the reference.
    with pytest.raises(RuntimeError, match="no CPU kernel"):
        ops.residual_rmsnorm_native(torch.ones(2, 3), torch.ones(2, 3), torch.ones(3), 0.0)


def test_softmax_and_attention_softmax_error_contract():
    for input, message in ((torch.tensor(1.0), "at least one dimension"), (torch.empty(2, 0), "non-empty final"),
                           (torch.ones(2, 3, dtype=torch.float16), "dtype torch.float32")):
        with pytest.raises(RuntimeError, match=message):
            ops.softmax_native(input)
    with pytest.raises(RuntimeError, match="inference-only"):
        ops.softmax_native(torch.ones(2, 3, requires_grad=True))
    scores = torch.ones((1, 2, 3, 4))
    mask = torch.zeros((1, 1, 3, 4))
    for bad_scores, bad_mask, scale, message in (
        (scores.reshape(2, 3, 4), mask, 0.5, "rank four"),
        (scores, torch.zeros((1, 1, 2, 4)), 0.5, "broadcastable"),
        (scores.half(), mask, 0.5, "scores must have dtype torch.float32"),
        (scores, mask, float("inf"), "finite FP32"),
    ):
        with pytest.raises(RuntimeError, match=message):
            ops.attention_score_softmax_native(bad_scores, bad_mask, scale)
    with pytest.raises(RuntimeError, match="inference-only"):
        ops.attention_score_softmax_native(scores.clone().requires_grad_(), mask, 0.5)


def test_rope_and_packed_swiglu_error_contract():
    q, k, c = _wave((2, 9, 7, 64)), _wave((2, 3, 7, 64)), _wave((2, 7, 64))
    for args, message in (
        ((q[0], k, c, c), "rank four"),
        ((q.double(), k, c, c), "float32"),
        ((q[..., :63], k[..., :63], c[..., :63], c[..., :63]), "even"),
        ((q, k[:1], c, c), "batch, sequence, and head dimensions must match"),
        ((q, k, c[:, :6], c[:, :6]), "not broadcastable"),
        ((q, k, c, c[:1]), "cos and sin shapes must match"),
    ):
        with pytest.raises(RuntimeError, match=message):
            ops.rope_native(*args)
    with pytest.raises(RuntimeError, match="inference-only"):
        ops.rope_native(q.clone().requires_grad_(), k, c, c)
    for packed, message in ((torch.tensor(1.0), "at least one dimension"), (torch.ones(2, 3), "must be even"),
                            (torch.ones(2, 4, dtype=torch.float64), "dtype torch.float32"),
                            (torch.ones(4, 2).t(), "must be contiguous")):
        with pytest.raises(RuntimeError, match=message):
            ops.packed_swiglu_native(packed)
    with pytest.raises(RuntimeError, match="inference-only"):
        ops.packed_swiglu_native(torch.ones(2, 4, requires_grad=True))


def _gqa_inputs(capacity: int = 17):
    g = torch.Generator().manual_seed(1307)
    return (torch.randn((1, 9, 1, 64), generator=g), torch.randn((1, 3, capacity, 64), generator=g),
            torch.randn((1, 3, capacity, 64), generator=g), torch.randn((1, 1, 1, capacity), generator=g) * 0.05)


def test_gqa_decode_error_contract():
    query, keys, values, mask = _gqa_inputs()
    cases = (
        ((query.expand(2, -1, -1, -1), keys.expand(2, -1, -1, -1), values.expand(2, -1, -1, -1),
          mask.expand(2, -1, -1, -1), 0.125, None), "batch size must be one"),
        ((query.half(), keys, values, mask, 0.125, None), "float32"),
        ((query, keys, values, mask[..., :-1], 0.125, None), "broadcastable"),
        ((query, keys, values, mask, 0.125, torch.tensor(18)), "within cache capacity"),
        ((query, keys, values, mask, 0.125, torch.tensor(0)), "within cache capacity"),
        ((query, keys, values, mask, float("nan"), None), "finite FP32"),
        ((query[:, :8], keys[:, :3], values[:, :3], None, 0.125, None), "divisible"),
        ((query, keys, values[..., :2, :], mask, 0.125, None), "shapes must match"),
    )
    for arguments, message in cases:
        with pytest.raises(RuntimeError, match=message):
            ops.gqa_decode_attention_native(*arguments)
    with pytest.raises(RuntimeError, match="inference-only"):
        ops.gqa_decode_attention_native(query.clone().requires_grad_(), keys, values, mask, 0.125)


def test_packed_qkv_rope_cache_and_gate_up_error_contract():
    packed, cos, keys = torch.ones(1, 1, 960), torch.ones(1, 1, 64), torch.ones(1, 3, 17, 64)
    length = torch.tensor(11)
    for args, message in (
        ((packed[..., :-1], cos, cos, keys, keys.clone(), length), r"\[1, 1, 960\]"),
        ((packed.double(), cos, cos, keys, keys.clone(), length), "float32"),
        ((packed, cos[..., :-1], cos, keys, keys.clone(), length), r"\[1, 1, 64\]"),
        ((packed, cos, cos, keys[:, :2], keys[:, :2].clone(), length), r"\[1, 3, capacity, 64\]"),
        ((packed, cos, cos, keys, keys.clone(), torch.tensor([11])), "scalar torch.int64"),
    ):
        with pytest.raises(RuntimeError, match=message):
            ops.packed_qkv_rope_cache_native(*args)
    with pytest.raises(RuntimeError, match="inference-only"):
        ops.packed_qkv_rope_cache_native(packed.clone().requires_grad_(), cos, cos, keys, keys.clone(), length)
    x, w, out = torch.ones(1, 1, 576), torch.ones(3072, 576), torch.empty(1, 1, 1536)
    for args, message in (((x[..., :-1], w, out), r"\[1, 1, 576\]"), ((x, w[:-1], out), r"\[3072, 576\]"),
                          ((x.double(), w, out), "float32"), ((x, w, out[..., :-1]), "output shape")):
        with pytest.raises(RuntimeError, match=message):
            ops.packed_gate_up_swiglu_native_out(*args)
    with pytest.raises(RuntimeError, match="inference-only"):
        ops.packed_gate_up_swiglu_native_out(x, w.clone().requires_grad_(), out)


def test_fake_tensor_contracts():
    with FakeTensorMode():
        hidden = torch.empty((2, 7, 576))
        norm, residual = ops.residual_rmsnorm_native(hidden, torch.empty_like(hidden), torch.empty(576), EPSILON)
        normed = ops.rms_norm_native(hidden, torch.empty(576), EPSILON)
        soft = ops.softmax_native(torch.empty((2, 9, 7, 129)))
        att = ops.attention_score_softmax_native(torch.empty((2, 9, 7, 129)), torch.empty((2, 1, 7, 129)), 0.125)
        swiglu = ops.packed_swiglu_native(torch.empty((2, 32, 3072)))
        q, k = ops.rope_native(torch.empty((2, 9, 7, 64)), torch.empty((2, 3, 7, 64)), torch.empty((1, 7, 64)),
                               torch.empty((1, 7, 64)))
        fake_keys = torch.empty((1, 3, 129, 64))
        gqa = ops.gqa_decode_attention_native(torch.empty((1, 9, 1, 64)), fake_keys, torch.empty_like(fake_keys),
                                              torch.empty((1, 1, 1, 129)), 0.125, torch.empty((), dtype=torch.int64))
        qkv = ops.packed_qkv_rope_cache_native(torch.empty((1, 1, 960)), torch.empty((1, 1, 64)),
                                               torch.empty((1, 1, 64)), torch.empty((1, 3, 17, 64)),
                                               torch.empty((1, 3, 17, 64)), torch.empty((), dtype=torch.int64))
        out = torch.empty((1, 1, 1536))
        gate_up = ops.packed_gate_up_swiglu_native_out(torch.empty((1, 1, 576)), torch.empty((3072, 576)), out)
    for tensor in (norm, residual, normed, soft, att, swiglu, q, k, gqa, qkv):
        assert isinstance(tensor, FakeTensor) and tensor.is_contiguous()
    assert norm is not residual and norm.shape == residual.shape == hidden.shape
    assert soft.shape == att.shape == (2, 9, 7, 129) and swiglu.shape == (2, 32, 1536)
    assert q.shape == (2, 9, 7, 64) and k.shape == (2, 3, 7, 64)
    assert gqa.shape == (1, 9, 1, 64) and qkv.shape == (1, 9, 1, 64)
    assert gate_up is out


def test_out_variant_workspace_shape_matches_reference():
    query, keys = torch.empty(1, 9, 1, 64), torch.empty(1, 3, 1024, 64)
    assert native_ops.gqa_decode_out_workspace_shape(query, keys) == (1, 9, 8, 66)


@pytest.mark.skipif(not _native.is_available(), reason="libflux_amd.so not built")
def test_gqa_decode_workspace_sizes():
    # head_dim 64 splits keys in chunks of 128, other head sizes in chunks of 256; one chunk needs no workspace.
    assert native_ops.gqa_decode_workspace_bytes(9, 128, 64) == 0
    assert native_ops.gqa_decode_workspace_bytes(9, 129, 64) == 9 * 2 * 66 * 4
    assert native_ops.gqa_decode_workspace_bytes(9, 8192, 64) == 9 * 64 * 66 * 4
    assert native_ops.gqa_decode_workspace_bytes(4, 256, 8) == 0
    assert native_ops.gqa_decode_workspace_bytes(4, 600, 8) == 4 * 3 * 10 * 4
    # The reference's out-variant workspace [1, Hq, ceil(capacity/128), D+2] always covers it.
    for capacity in (513, 1024, 8192, 16384):
        shape = native_ops.gqa_decode_out_workspace_shape(torch.empty(1, 9, 1, 64), torch.empty(1, 3, capacity, 64))
        assert math.prod(shape) * 4 >= native_ops.gqa_decode_workspace_bytes(9, capacity, 64)
    with pytest.raises(RuntimeError, match="invalid argument"):
        native_ops.gqa_decode_workspace_bytes(9, 16385, 64)
