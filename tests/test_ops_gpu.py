"""GPU parity of the ``torch.ops.flux`` eager operators (HIP kernels through
the C ABI) against the CPU oracle (float64) and, where the reference's own
tests use them, PyTorch fp32 on the GPU; plus the out-variant identity,
opcheck contracts and the Flux eager model against Hugging Face.

Tolerances are the reference's (tests/test_ops.py:103-580): RMSNorm rtol 1e-5
atol 2e-6, softmax rtol 1e-5 atol 5e-7, SwiGLU rtol/atol 2e-6, GQA decode rtol
2e-5 atol 1e-6; RoPE and the packed QKV cache step are bit-exact.
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F
from transformers import LlamaConfig, LlamaForCausalLM, StaticCache
from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

from flux_amd import ops
from flux_amd.model import smollm2_flux
from oracle import kernels as ref

pytestmark = pytest.mark.gpu
EPSILON = 1e-5


def _wave(shape, device):
    values = torch.arange(math.prod(shape), device=device, dtype=torch.float32)
    return (torch.sin(values * 0.013) + torch.cos(values * 0.007)).reshape(shape)


def _opcheck(op, args, **kwargs):
    result = torch.library.opcheck(op, args, **kwargs)
    assert all(status == "SUCCESS" for status in result.values()), result


# --------------------------------------------------------------------------- RMSNorm

def test_rmsnorm_layout_and_oracle(gpu_device):
    input = _wave((2, 576, 7), gpu_device).transpose(1, 2)
    weight = torch.linspace(0.25, 1.75, 1152, device=gpu_device)[::2]
    assert not input.is_contiguous() and not weight.is_contiguous()
    actual = ops.rms_norm_native(input, weight, EPSILON)
    assert actual.shape == input.shape and actual.is_contiguous() and actual.device == input.device
    expected = ref.rmsnorm(input.cpu(), weight.cpu(), EPSILON)
    torch.testing.assert_close(actual.cpu().double(), expected, rtol=1e-5, atol=2e-6)
    for cols in (1, 3, 577, 4096):
        x = _wave((5, cols), gpu_device) * 3.0
        w = torch.linspace(0.5, 1.5, cols, device=gpu_device)
        torch.testing.assert_close(ops.rms_norm_native(x, w, EPSILON).cpu().double(),
                                   ref.rmsnorm(x.cpu(), w.cpu(), EPSILON), rtol=1e-5, atol=2e-6)


def test_rmsnorm_out_identity_alias_and_opcheck(gpu_device):
    input = _wave((2, 7, 576), gpu_device)
    weight = torch.linspace(0.25, 1.75, 576, device=gpu_device)
    output = torch.full_like(input, 73.0)
    assert ops.rms_norm_native_out(input, weight, EPSILON, output) is output
    torch.testing.assert_close(output.cpu().double(), ref.rmsnorm(input.cpu(), weight.cpu(), EPSILON),
                               rtol=1e-5, atol=2e-6)
    with pytest.raises(RuntimeError, match="must not alias"):
        ops.rms_norm_native_out(input, weight, EPSILON, input)
    _opcheck(torch.ops.flux.rmsnorm.default, (input, torch.ones(576, device=gpu_device), EPSILON),
             rtol=1e-5, atol=2e-6)
    _opcheck(torch.ops.flux.rmsnorm_out.default, (input, weight, EPSILON, output),
             test_utils=("test_schema", "test_faketensor"))


def test_residual_rmsnorm_and_out(gpu_device):
    hidden = _wave((2, 7, 576), gpu_device)
    residual = _wave((2, 7, 576), gpu_device).mul_(0.25)
    weight = torch.linspace(0.25, 1.75, 576, device=gpu_device)
    before = hidden.clone()
    norm, res = ops.residual_rmsnorm_native(hidden, residual, weight, EPSILON)
    assert norm.is_contiguous() and res.is_contiguous() and norm.data_ptr() != res.data_ptr()
    assert torch.equal(hidden, before)
    expected_norm, expected_res = ref.residual_rmsnorm(hidden.cpu(), residual.cpu(), weight.cpu(), EPSILON)
    assert torch.equal(res.cpu(), expected_res)
    torch.testing.assert_close(norm.cpu().double(), expected_norm, rtol=1e-5, atol=2e-6)
    norm_out = torch.full_like(hidden, 41.0)
    res_out = torch.full_like(hidden, -41.0)
    returned = ops.residual_rmsnorm_native_out(hidden, residual, weight, EPSILON, norm_out, res_out)
    assert returned[0] is norm_out and returned[1] is res_out
    assert torch.equal(norm_out, norm) and torch.equal(res_out, res)
    with pytest.raises(RuntimeError, match="must not alias each other"):
        ops.residual_rmsnorm_native_out(hidden, residual, weight, EPSILON, norm_out, norm_out)
    _opcheck(torch.ops.flux.residual_rmsnorm.default, (hidden, residual, torch.ones(576, device=gpu_device), EPSILON),
             rtol=1e-5, atol=2e-6)


# --------------------------------------------------------------------------- softmax

@pytest.mark.parametrize("width", [1, 17, 64, 65, 129, 256, 300, 512, 1000, 1024, 1025, 2048, 3000, 4096, 8192,
                                   8193, 20000])
def test_softmax_every_width_tier(gpu_device, width):
    input = 3.0 * _wave((5, width), gpu_device)
    actual = ops.softmax_native(input)
    assert actual.shape == input.shape and actual.is_contiguous()
    torch.testing.assert_close(actual.cpu().double(), ref.softmax_rows(input.cpu()), rtol=1e-5, atol=5e-7)


def test_softmax_layout_masks_and_opcheck(gpu_device):
    input = 3.0 * _wave((7, 2, 129), gpu_device).transpose(0, 1)
    torch.testing.assert_close(ops.softmax_native(input).cpu().double(), ref.softmax_rows(input.cpu()), rtol=1e-5,
                               atol=5e-7)
    masked = torch.tensor([[0.0, float("-inf"), 1.0, float("-inf")]], device=gpu_device)
    out = ops.softmax_native(masked).cpu()
    assert out[0, 1] == 0 and out[0, 3] == 0
    _opcheck(torch.ops.flux.softmax.default, (_wave((2, 7, 129), gpu_device),), rtol=1e-5, atol=5e-7)


@pytest.mark.parametrize("mask_shape", [(2, 1, 5, 17), (1, 3, 1, 17), (1, 1, 1, 1), (2, 3, 5, 17), (1, 1, 5, 1)])
def test_attention_score_softmax_broadcasts(gpu_device, mask_shape):
    scores = 3.0 * _wave((2, 3, 5, 17), gpu_device)
    mask = _wave(mask_shape, gpu_device) * 0.25
    actual = ops.attention_score_softmax_native(scores, mask, 17 ** -0.5)
    assert actual.shape == scores.shape and actual.is_contiguous()
    expected = ref.attention_score_softmax(scores.cpu(), mask.cpu(), 17 ** -0.5)
    torch.testing.assert_close(actual.cpu().double(), expected, rtol=1e-5, atol=5e-7)
    torch.testing.assert_close(actual, torch.softmax(scores * (17 ** -0.5) + mask, dim=-1), rtol=1e-5, atol=5e-7)


@pytest.mark.parametrize("seq", [9, 300, 1500, 5000])
@pytest.mark.parametrize("pad", [0, 7])
def test_attention_score_softmax_causal_strided_mask(gpu_device, seq, pad):
    """HF's eager causal mask (finfo.min above the diagonal), contiguous or sliced from a wider mask."""
    g = torch.Generator(device=gpu_device).manual_seed(seq)
    scores = torch.randn((1, 2, seq, seq), generator=g, device=gpu_device) * 4.0
    full = torch.full((seq, seq + pad), torch.finfo(torch.float32).min, device=gpu_device).triu(1)
    mask = full[None, None, :, :seq]
    assert mask.is_contiguous() == (pad == 0)
    actual = ops.attention_score_softmax_native(scores, mask, 0.125)
    expected = ref.attention_score_softmax(scores.cpu(), mask.cpu(), 0.125)
    torch.testing.assert_close(actual.cpu().double(), expected, rtol=1e-5, atol=5e-7)


def test_attention_score_softmax_opcheck(gpu_device):
    _opcheck(torch.ops.flux.attention_score_softmax.default,
             (_wave((2, 3, 4, 17), gpu_device), _wave((2, 1, 4, 17), gpu_device), 0.125), rtol=1e-5, atol=5e-7)


# --------------------------------------------------------------------------- RoPE

def _rope_inputs(device, dim=64, heads=(9, 3)):
    hidden = _wave((2, 7, heads[0] * dim), device)
    query = hidden.view(2, 7, heads[0], dim).transpose(1, 2)
    key = hidden[..., :heads[1] * dim].view(2, 7, heads[1], dim).transpose(1, 2)
    positions = torch.arange(31, 38, device=device, dtype=torch.float32)
    inv_freq = 1.0 / 100000.0 ** (torch.arange(0, dim, 2, device=device).float() / dim)
    frequencies = torch.outer(positions, inv_freq)
    embedding = torch.cat((frequencies, frequencies), dim=-1)
    return query, key, embedding.cos().unsqueeze(0).expand(2, -1, -1), embedding.sin().unsqueeze(0).expand(2, -1, -1)


@pytest.mark.parametrize("dim,heads", [(64, (9, 3)), (8, (4, 2)), (128, (2, 2)), (6, (2, 1))])
def test_rope_bit_exact_vs_transformers(gpu_device, dim, heads):
    inputs = _rope_inputs(gpu_device, dim, heads)
    actual = ops.rope_native(*inputs)
    expected = apply_rotary_pos_emb(*inputs)
    assert actual[0].is_contiguous() and actual[1].is_contiguous()
    assert torch.equal(actual[0], expected[0]) and torch.equal(actual[1], expected[1])
    # Broadcast cos/sin batch (rope_batch == 1) and the oracle's float32 rounding.
    query, key, cos, sin = inputs
    q1, k1 = ops.rope_native(query, key, cos[:1], sin[:1])
    assert torch.equal(q1, actual[0]) and torch.equal(k1, actual[1])
    oracle_q = ref.rope_rows(query[0].cpu(), cos[0].cpu(), sin[0].cpu())
    assert torch.equal(actual[0][0].cpu(), oracle_q)
    # Contiguous inputs take the float4 path when head_dim % 8 == 0; the result is the same.
    qc, kc = ops.rope_native(query.contiguous(), key.contiguous(), cos.contiguous(), sin.contiguous())
    assert torch.equal(qc, actual[0]) and torch.equal(kc, actual[1])


def test_rope_opcheck(gpu_device):
    with torch.inference_mode():
        _opcheck(torch.ops.flux.rope.default, _rope_inputs(gpu_device), rtol=1e-6, atol=2e-7)


# --------------------------------------------------------------------------- packed SwiGLU

@pytest.mark.parametrize("shape", [(1, 7, 3072), (2, 5, 6), (3, 2), (4, 1538)])
def test_packed_swiglu(gpu_device, shape):
    packed = _wave(shape, gpu_device) * 4.0
    gate, up = packed.chunk(2, dim=-1)
    actual = ops.packed_swiglu_native(packed)
    assert actual.shape == (*shape[:-1], shape[-1] // 2) and actual.is_contiguous()
    torch.testing.assert_close(actual, F.silu(gate) * up, rtol=2e-6, atol=2e-6)
    torch.testing.assert_close(actual.cpu().double(), ref.packed_swiglu(packed.cpu()), rtol=2e-6, atol=2e-6)


def test_packed_swiglu_out_and_opcheck(gpu_device):
    packed = _wave((2, 7, 3072), gpu_device)
    output = torch.full((2, 7, 1536), 59.0, device=gpu_device)
    assert ops.packed_swiglu_native_out(packed, output) is output
    gate, up = packed.chunk(2, dim=-1)
    torch.testing.assert_close(output, F.silu(gate) * up, rtol=2e-6, atol=2e-6)
    with pytest.raises(RuntimeError, match="output shape"):
        ops.packed_swiglu_native_out(packed, output[..., :-1])
    _opcheck(torch.ops.flux.packed_swiglu.default, (packed,), rtol=2e-6, atol=2e-6)


# --------------------------------------------------------------------------- GQA decode attention

def _gqa_inputs(device, capacity=73, heads=(9, 3), dim=64, seed=1307):
    g = torch.Generator(device=device).manual_seed(seed)
    query = torch.randn((1, heads[0], 1, dim), generator=g, device=device)
    keys = torch.randn((1, heads[1], capacity, dim), generator=g, device=device)
    values = torch.randn((1, heads[1], capacity, dim), generator=g, device=device)
    mask = torch.randn((1, 1, 1, capacity), generator=g, device=device) * 0.05
    return query, keys, values, mask


def _gqa_oracle(query, keys, values, mask, scale, length):
    hq = query.shape[1]
    m = None if mask is None else mask.cpu().expand(1, hq, 1, keys.shape[2])[0, :, 0]
    out = ref.gqa_decode_attention(query[0, :, 0].cpu(), keys[0].cpu(), values[0].cpu(), length, scale, m)
    return out.view(1, hq, 1, -1)


@pytest.mark.parametrize("capacity,length", [(73, 41), (73, 73), (256, 256), (257, 257), (257, 1), (1024, 777),
                                             (8192, 8192), (8192, 3), (16384, 12345)])
def test_gqa_decode_lengths_and_mask(gpu_device, capacity, length):
    query, keys, values, mask = _gqa_inputs(gpu_device, capacity)
    cache_length = torch.tensor(length, device=gpu_device)
    actual = ops.gqa_decode_attention_native(query, keys, values, mask, 0.125, cache_length)
    assert actual.shape == query.shape and actual.is_contiguous()
    torch.testing.assert_close(actual.cpu().double(), _gqa_oracle(query, keys, values, mask, 0.125, length),
                               rtol=2e-5, atol=1e-6)
    plain = ops.gqa_decode_attention_native(query, keys, values, None, 0.125, cache_length)
    torch.testing.assert_close(plain.cpu().double(), _gqa_oracle(query, keys, values, None, 0.125, length),
                               rtol=2e-5, atol=1e-6)


@pytest.mark.parametrize("heads,dim", [((4, 2), 8), ((8, 8), 128), ((6, 1), 36), ((9, 3), 66)])
def test_gqa_decode_general_geometry(gpu_device, heads, dim):
    query, keys, values, _ = _gqa_inputs(gpu_device, 600, heads, dim)
    mask = torch.randn((1, heads[0], 1, 600), device=gpu_device)
    actual = ops.gqa_decode_attention_native(query, keys, values, mask, dim ** -0.5)
    torch.testing.assert_close(actual.cpu().double(), _gqa_oracle(query, keys, values, mask, dim ** -0.5, 600),
                               rtol=2e-5, atol=1e-6)


def test_gqa_decode_strided_caches_and_clamped_length(gpu_device):
    g = torch.Generator(device=gpu_device).manual_seed(5)
    query = torch.randn((1, 1, 9, 64), generator=g, device=gpu_device).transpose(1, 2)  # [1, 9, 1, 64] strided
    storage = torch.randn((1, 700, 3, 64), generator=g, device=gpu_device)
    keys = storage.transpose(1, 2)                      # strides (.., 64, 192, 1)
    values = torch.randn((1, 3, 700, 128), generator=g, device=gpu_device)[..., ::2]  # dimension stride 2
    assert not keys.is_contiguous() and not values.is_contiguous()
    expected = _gqa_oracle(query, keys, values, None, 0.125, 650)
    actual = ops.gqa_decode_attention_native(query, keys, values, None, 0.125, torch.tensor(650, device=gpu_device))
    torch.testing.assert_close(actual.cpu().double(), expected, rtol=2e-5, atol=1e-6)
    # The device kernel clamps the length into [1, capacity] (as the reference's CUDA path does).
    low = ops.gqa_decode_attention_native(query, keys, values, None, 0.125, torch.tensor(0, device=gpu_device))
    torch.testing.assert_close(low.cpu().double(), _gqa_oracle(query, keys, values, None, 0.125, 1),
                               rtol=2e-5, atol=1e-6)
    high = ops.gqa_decode_attention_native(query, keys, values, None, 0.125, torch.tensor(9999, device=gpu_device))
    torch.testing.assert_close(high.cpu().double(), _gqa_oracle(query, keys, values, None, 0.125, 700),
                               rtol=2e-5, atol=1e-6)
    full = ops.gqa_decode_attention_native(query, keys, values, None, 0.125)
    assert torch.equal(full, high)


def test_gqa_decode_out_identity_and_opcheck(gpu_device):
    query, keys, values, mask = _gqa_inputs(gpu_device, 1024)
    length = torch.tensor(777, device=gpu_device)
    output = torch.full_like(query, 67.0)
    workspace = torch.empty((1, 9, 8, 66), device=gpu_device)
    assert ops.gqa_decode_attention_native_out(query, keys, values, mask, 0.125, length, output, workspace) is output
    torch.testing.assert_close(output.cpu().double(), _gqa_oracle(query, keys, values, mask, 0.125, 777),
                               rtol=2e-5, atol=1e-6)
    with pytest.raises(RuntimeError, match="workspace shape"):
        ops.gqa_decode_attention_native_out(query, keys, values, mask, 0.125, length, output, workspace[:, :, :7])
    small = _gqa_inputs(gpu_device, 17)
    _opcheck(torch.ops.flux.gqa_decode_attention.default,
             (*small, 0.125, torch.tensor(11, device=gpu_device)), rtol=2e-5, atol=1e-6)


# --------------------------------------------------------------------------- packed QKV / RoPE / cache

def _qkv_inputs(device, capacity=17, length=11):
    g = torch.Generator(device=device).manual_seed(1245)
    packed = torch.randn((1, 1, 960), generator=g, device=device)
    frequencies = torch.randn((1, 1, 64), generator=g, device=device)
    keys = torch.randn((1, 3, capacity, 64), generator=g, device=device)
    values = torch.randn((1, 3, capacity, 64), generator=g, device=device)
    return packed, frequencies.cos(), frequencies.sin(), keys, values, torch.tensor(length, device=device)


def _qkv_expected(inputs):
    packed, cos, sin, keys, values, length = inputs
    position = int(length.item())
    query = packed[..., :576].view(1, 1, 9, 64).transpose(1, 2)
    key = packed[..., 576:768].view(1, 1, 3, 64).transpose(1, 2)
    value = packed[..., 768:].view(1, 1, 3, 64).transpose(1, 2)
    query, key = apply_rotary_pos_emb(query, key, cos, sin)
    expected_keys, expected_values = keys.clone(), values.clone()
    expected_keys[..., position:position + 1, :].copy_(key)
    expected_values[..., position:position + 1, :].copy_(value)
    return query, expected_keys, expected_values


def test_packed_qkv_rope_cache_bit_exact(gpu_device):
    inputs = _qkv_inputs(gpu_device)
    expected_query, expected_keys, expected_values = _qkv_expected(inputs)
    actual = ops.packed_qkv_rope_cache_native(*inputs)
    assert actual.shape == (1, 9, 1, 64) and actual.is_contiguous()
    assert inputs[-1].item() == 12
    assert torch.equal(actual, expected_query)
    assert torch.equal(inputs[3], expected_keys) and torch.equal(inputs[4], expected_values)
    out_inputs = _qkv_inputs(gpu_device)
    output = torch.full((1, 9, 1, 64), 83.0, device=gpu_device)
    assert ops.packed_qkv_rope_cache_native_out(*out_inputs, output) is output
    assert torch.equal(output, expected_query) and torch.equal(out_inputs[3], expected_keys)


def test_packed_qkv_rope_cache_out_of_range_and_strided(gpu_device):
    inputs = _qkv_inputs(gpu_device, capacity=17, length=17)
    keys_before, values_before = inputs[3].clone(), inputs[4].clone()
    output = torch.full((1, 9, 1, 64), 83.0, device=gpu_device)
    ops.packed_qkv_rope_cache_native_out(*inputs, output)
    assert inputs[-1].item() == 17 and torch.all(output == 83.0)
    assert torch.equal(inputs[3], keys_before) and torch.equal(inputs[4], values_before)
    # Caches laid out [1, capacity, 3, 64] and viewed as [1, 3, capacity, 64].
    packed, cos, sin, keys, values, _ = _qkv_inputs(gpu_device, capacity=600, length=0)
    k_store = keys.transpose(1, 2).contiguous()
    v_store = values.transpose(1, 2).contiguous()
    length = torch.tensor(599, device=gpu_device)
    expected_query, expected_keys, expected_values = _qkv_expected((packed, cos, sin, keys, values, length))
    query = ops.packed_qkv_rope_cache_native(packed, cos, sin, k_store.transpose(1, 2), v_store.transpose(1, 2),
                                             length)
    assert torch.equal(query, expected_query) and length.item() == 600
    assert torch.equal(k_store.transpose(1, 2), expected_keys)
    assert torch.equal(v_store.transpose(1, 2), expected_values)


def test_packed_qkv_rope_cache_opcheck(gpu_device):
    with torch.inference_mode():
        _opcheck(torch.ops.flux.packed_qkv_rope_cache.default, _qkv_inputs(gpu_device), rtol=0, atol=0)


# --------------------------------------------------------------------------- decode GEMV operators

def test_packed_gate_up_swiglu_out(gpu_device):
    g = torch.Generator(device=gpu_device).manual_seed(1234)
    input = torch.randn((1, 1, 576), generator=g, device=gpu_device)
    weight = torch.randn((3072, 576), generator=g, device=gpu_device)
    output = torch.full((1, 1, 1536), float("nan"), device=gpu_device)
    assert ops.packed_gate_up_swiglu_native_out(input, weight, output) is output
    packed = F.linear(input, weight)
    torch.testing.assert_close(output, F.silu(packed[..., :1536]) * packed[..., 1536:], rtol=1e-4, atol=1e-3)
    expected = ref.gate_up_swiglu(input[0, 0].cpu(), weight.cpu())
    torch.testing.assert_close(output[0, 0].cpu().double(), expected, rtol=1e-5, atol=1e-4)
    _opcheck(torch.ops.flux.packed_gate_up_swiglu_out.default, (input, weight, output),
             test_utils=("test_schema", "test_faketensor"))


@pytest.mark.parametrize("rows", [960, 576])
def test_decode_projection_out(gpu_device, rows):
    g = torch.Generator(device=gpu_device).manual_seed(rows)
    input = torch.randn((1, 1, 576), generator=g, device=gpu_device)
    weight = torch.randn((rows, 576), generator=g, device=gpu_device)
    output = torch.full((1, 1, rows), float("nan"), device=gpu_device)
    assert ops.decode_projection_out(input, weight, output) is output
    expected = weight.cpu().double() @ input[0, 0].cpu().double()
    torch.testing.assert_close(output[0, 0].cpu().double(), expected, rtol=1e-5, atol=1e-4)


# --------------------------------------------------------------------------- Flux eager model

def _llama(config: LlamaConfig, device) -> LlamaForCausalLM:
    torch.manual_seed(1234)
    model = LlamaForCausalLM(config).float().eval().to(device)
    with torch.no_grad():  # non-trivial norms so a swapped weight would show
        for name, p in model.named_parameters():
            if "norm" in name:
                p.copy_(1.0 + 0.1 * torch.randn_like(p))
    return model


def _tiny_config() -> LlamaConfig:
    config = LlamaConfig(hidden_size=32, intermediate_size=64, num_hidden_layers=2, num_attention_heads=4,
                         num_key_value_heads=2, head_dim=8, vocab_size=128, max_position_embeddings=64,
                         rms_norm_eps=1e-5, attention_bias=False, attention_dropout=0.0, mlp_bias=False)
    config._attn_implementation = "eager"
    return config


def _smol_config(layers: int = 2, vocab: int = 256) -> LlamaConfig:
    config = LlamaConfig(hidden_size=576, intermediate_size=1536, num_hidden_layers=layers, num_attention_heads=9,
                         num_key_value_heads=3, head_dim=64, vocab_size=vocab, max_position_embeddings=8192,
                         rms_norm_eps=1e-5, rope_theta=100000.0, attention_bias=False, attention_dropout=0.0,
                         mlp_bias=False, tie_word_embeddings=True)
    config._attn_implementation = "eager"
    return config


def _counting(monkeypatch, names):
    counts = {name: 0 for name in names}
    for name in names:
        original = getattr(smollm2_flux, name)

        def wrapper(*args, _original=original, _name=name, **kwargs):
            counts[_name] += 1
            return _original(*args, **kwargs)

        monkeypatch.setattr(smollm2_flux, name, wrapper)
    return counts


def test_flux_eager_model_matches_hf_dynamic_cache(gpu_device, monkeypatch):
    reference = _llama(_tiny_config(), gpu_device)
    flux = _llama(_tiny_config(), gpu_device)
    smollm2_flux.enable_flux_ops(flux, operators=smollm2_flux.FINAL_FLUX_OPERATOR_CATEGORIES)
    counts = _counting(monkeypatch, ["rms_norm_native", "residual_rmsnorm_native", "rope_native",
                                     "attention_score_softmax_native", "packed_swiglu_native",
                                     "gqa_decode_attention_native"])
    ids = ((torch.arange(9).unsqueeze(0) * 11 + 3) % 128).to(gpu_device)
    with torch.inference_mode():
        torch.testing.assert_close(flux(input_ids=ids).logits, reference(input_ids=ids).logits, rtol=2e-4,
                                   atol=2e-5)
        generated_ref = reference.generate(input_ids=ids, do_sample=False, max_new_tokens=6, pad_token_id=0)
        generated = flux.generate(input_ids=ids, do_sample=False, max_new_tokens=6, pad_token_id=0)
    assert torch.equal(generated, generated_ref)
    assert all(counts[n] > 0 for n in counts), counts


def test_flux_eager_model_static_cache_fused_decode(gpu_device, monkeypatch):
    """SmolLM2 geometry with a StaticCache of capacity 1024: one-token steps take
    flux::packed_qkv_rope_cache + flux::gqa_decode_attention (reference :437-600)."""
    config = _smol_config()
    reference = _llama(config, gpu_device)
    flux = _llama(config, gpu_device)
    smollm2_flux.enable_flux_ops(flux, operators=smollm2_flux.FINAL_FLUX_OPERATOR_CATEGORIES)
    counts = _counting(monkeypatch, ["packed_qkv_rope_cache_native", "gqa_decode_attention_native",
                                     "attention_score_softmax_native"])
    ids = ((torch.arange(13).unsqueeze(0) * 37 + 5) % 256).to(gpu_device)

    def greedy(model, steps=8):
        cache = StaticCache(config=model.config, max_cache_len=1024)
        tokens, logits = [], []
        with torch.inference_mode():
            out = model(input_ids=ids, past_key_values=cache, use_cache=True)
            for _ in range(steps):
                step_logits = out.logits[:, -1]
                logits.append(step_logits.clone())
                token = step_logits.argmax(-1, keepdim=True)
                tokens.append(int(token))
                out = model(input_ids=token, past_key_values=cache, use_cache=True)
        return tokens, torch.stack(logits)

    expected_tokens, expected_logits = greedy(reference)
    tokens, logits = greedy(flux)
    assert tokens == expected_tokens
    torch.testing.assert_close(logits, expected_logits, rtol=1e-4, atol=1e-4)
    layers = config.num_hidden_layers
    assert counts["packed_qkv_rope_cache_native"] == 8 * layers
    assert counts["gqa_decode_attention_native"] == 8 * layers
    assert counts["attention_score_softmax_native"] == layers
