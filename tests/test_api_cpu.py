"""Python surface checks on the CPU (no GPU): enable_flux_ops wiring, packed
parameters, state-dict transparency, the GPU-only contract of the enabled
model, and the runtime's input validation that happens before the native
boundary.

Mirrors tests/test_system.py:136-292 of the reference (module replacement and
HF equivalence on a small model, state-dict round trip, error contract)."""

from __future__ import annotations

import pytest
import torch
from transformers import LlamaConfig, LlamaForCausalLM

from flux_amd.model import smollm2_flux
from flux_amd.runtime import NativeSmolLM2Decode, NativeSmolLM2Prefill, native_smollm2_greedy_generate


def _config(layers: int = 2) -> LlamaConfig:
    config = LlamaConfig(hidden_size=32, intermediate_size=64, num_hidden_layers=layers, num_attention_heads=4,
                         num_key_value_heads=2, head_dim=8, vocab_size=128, max_position_embeddings=64,
                         rms_norm_eps=1e-5, attention_bias=False, attention_dropout=0.0, mlp_bias=False)
    config._attn_implementation = "eager"
    return config


def _model(layers: int = 2) -> LlamaForCausalLM:
    torch.manual_seed(1234)
    return LlamaForCausalLM(_config(layers)).float().eval()


def test_final_configuration_is_the_complete_retained_set():
    assert smollm2_flux.FINAL_FLUX_OPERATOR_CATEGORIES == {
        "rmsnorm", "residual_rmsnorm", "rope", "softmax", "gqa_decode_attention", "mlp", "packed_swiglu", "qkv",
        "packed_qkv_rope_cache", "cublaslt_projection", "fused_gate_up_swiglu"}


@pytest.mark.parametrize("operators,message", [
    ({"bogus"}, "unknown Flux operator categories"),
    (set(), "at least one"),
    ({"packed_swiglu"}, '"packed_swiglu" requires the "mlp"'),
    ({"packed_qkv_rope_cache", "rope"}, '"packed_qkv_rope_cache" requires'),
    ({"cublaslt_projection", "rope"}, '"cublaslt_projection" requires'),
    ({"fused_gate_up_swiglu", "mlp"}, '"fused_gate_up_swiglu" requires'),
])
def test_category_dependency_errors(operators, message):
    with pytest.raises(ValueError, match=message):
        smollm2_flux.enable_flux_ops(_model(), operators=operators)


def test_model_errors():
    model = _model()
    model.train()
    with pytest.raises(ValueError, match="inference-only"):
        smollm2_flux.enable_flux_ops(model)
    with pytest.raises(TypeError, match="LlamaForCausalLM"):
        smollm2_flux.enable_flux_ops(torch.nn.Linear(2, 2))
    model = _model().double()
    with pytest.raises(TypeError, match="float32"):
        smollm2_flux.enable_flux_ops(model)
    model = _model()
    smollm2_flux.enable_flux_ops(model)
    with pytest.raises(ValueError, match="already enabled"):
        smollm2_flux.enable_flux_ops(model)


def test_missing_native_library_fails_loudly(monkeypatch):
    monkeypatch.setattr(smollm2_flux, "native_library_is_available", lambda: False)
    with pytest.raises(RuntimeError, match="not built"):
        smollm2_flux.enable_flux_ops(_model())


def test_packed_parameters_and_equivalence():
    reference = _model()
    flux = _model()
    flux.load_state_dict(reference.state_dict())
    smollm2_flux.enable_flux_ops(flux, operators=smollm2_flux.FINAL_FLUX_OPERATOR_CATEGORIES)
    counts = smollm2_flux.flux_operator_counts(flux)
    assert counts["decoder_layers"] == 2 and counts["packed_qkv_modules"] == 2 and counts["packed_mlp_modules"] == 2
    for ref_layer, layer in zip(reference.model.layers, flux.model.layers):
        attn = ref_layer.self_attn
        expected_qkv = torch.cat((attn.q_proj.weight, attn.k_proj.weight, attn.v_proj.weight), dim=0)
        assert torch.equal(layer.self_attn.packed_qkv.weight, expected_qkv)
        mlp = ref_layer.mlp
        assert torch.equal(layer.mlp.gate_up_proj.weight, torch.cat((mlp.gate_proj.weight, mlp.up_proj.weight)))
    assert flux._flux_operator_categories == tuple(sorted(smollm2_flux.FINAL_FLUX_OPERATOR_CATEGORIES))
    # The Flux operators have no CPU kernel: an enabled model computes on GPU
    # tensors only (the HF-equivalence check is tests/test_ops_gpu.py).
    ids = (torch.arange(9).unsqueeze(0) * 11 + 3) % 128
    with torch.inference_mode(), pytest.raises(RuntimeError, match="no CPU kernel"):
        flux(input_ids=ids)


def test_state_dict_keeps_hf_keys_and_round_trips(tmp_path):
    reference = _model()
    flux = _model()
    flux.load_state_dict(reference.state_dict())
    smollm2_flux.enable_flux_ops(flux, operators=smollm2_flux.FINAL_FLUX_OPERATOR_CATEGORIES)
    state = flux.state_dict()
    assert not any("packed_qkv" in k or "gate_up_proj" in k for k in state)
    for key, value in reference.state_dict().items():
        assert torch.equal(state[key], value), key
    flux.save_pretrained(tmp_path)
    restored = LlamaForCausalLM.from_pretrained(tmp_path, attn_implementation="eager").float().eval()
    for key, value in reference.state_dict().items():
        assert torch.equal(restored.state_dict()[key], value), key
    # Loading HF keys into an enabled model packs them again.
    other = _model(2)
    smollm2_flux.enable_flux_ops(other, operators=smollm2_flux.FINAL_FLUX_OPERATOR_CATEGORIES)
    other.load_state_dict(reference.state_dict())
    assert torch.equal(other.model.layers[0].mlp.gate_up_proj.weight, flux.model.layers[0].mlp.gate_up_proj.weight)


def test_runtime_input_validation_before_native_boundary():
    model = _model()
    smollm2_flux.enable_flux_ops(model, operators=smollm2_flux.FINAL_FLUX_OPERATOR_CATEGORIES)
    ids = (torch.arange(5).unsqueeze(0) * 11 + 3) % 128
    with pytest.raises(TypeError, match="capture"):
        NativeSmolLM2Prefill()
    with pytest.raises(TypeError, match="capture"):
        NativeSmolLM2Decode()
    with pytest.raises(ValueError, match="non-negative"):
        NativeSmolLM2Prefill.capture(model, ids, max_decode_steps=-1)
    with pytest.raises(ValueError, match="batch of one"):
        NativeSmolLM2Prefill.capture(model, ids.expand(2, -1))
    with pytest.raises(ValueError, match="rank-2"):
        NativeSmolLM2Prefill.capture(model, ids[0])
    with pytest.raises(ValueError, match="contiguous"):
        NativeSmolLM2Prefill.capture(model, ids.repeat(1, 2)[:, ::2])
    with pytest.raises(ValueError, match="position limit"):
        NativeSmolLM2Prefill.capture(model, ids, max_decode_steps=1000)
    with pytest.raises(ValueError, match="max_new_tokens"):
        native_smollm2_greedy_generate(model, ids, max_new_tokens=0)
    with pytest.raises(ValueError, match="max_decode_steps must be positive"):
        NativeSmolLM2Decode.capture(model, ids, max_decode_steps=0)
    if not torch.cuda.is_available():
        with pytest.raises(RuntimeError, match="ROCm GPU"):
            NativeSmolLM2Prefill.capture(model, ids, max_decode_steps=2)


def test_geometry_and_category_validation_order():
    """After device checks, geometry and category errors name the retained configuration."""
    if torch.cuda.is_available():
        pytest.skip("exercised on CPU only")
    model = _model()
    ids = (torch.arange(3).unsqueeze(0) * 11 + 3) % 128
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        NativeSmolLM2Decode._validate_model_and_state(model, ids[:, :1], [], [], cache_position=0, cache_capacity=4)


def test_layer_decode_requires_gpu_tensors():
    from flux_amd.runtime import NativeSmolLM2LayerDecode

    hidden = torch.zeros(1, 1, 576)
    with pytest.raises(RuntimeError, match="initial_hidden must be a CUDA tensor"):
        NativeSmolLM2LayerDecode(hidden, torch.ones(576), torch.zeros(960, 576), torch.zeros(576, 576),
                                 torch.ones(576), torch.zeros(3072, 576), torch.zeros(576, 1536), torch.zeros(8, 64),
                                 torch.zeros(8, 64), torch.zeros(1, 3, 0, 64), torch.zeros(1, 3, 0, 64), 8, 0, 1e-5,
                                 0.125)


def test_audit_argument_validation():
    from flux_amd.runtime.audit import runtime_audit

    with pytest.raises(ValueError, match="audit capacity must exceed audit replays plus three warmups"):
        runtime_audit(_model(), capacity=10, replays=7)


def _smol_geometry_model(vocab: int = 64) -> LlamaForCausalLM:
    """SmolLM2 geometry (30 layers) on the meta device is too large to build per test on the CPU;
    two of its layers suffice for the per-tensor checks, which iterate over model.model.layers."""
    config = LlamaConfig(hidden_size=576, intermediate_size=1536, num_hidden_layers=2, num_attention_heads=9,
                         num_key_value_heads=3, head_dim=64, vocab_size=vocab, max_position_embeddings=64,
                         rms_norm_eps=1e-5, attention_bias=False, attention_dropout=0.0, mlp_bias=False,
                         tie_word_embeddings=True)
    config._attn_implementation = "eager"
    torch.manual_seed(7)
    model = LlamaForCausalLM(config).float().eval()
    return smollm2_flux.enable_flux_ops(model, operators=smollm2_flux.FINAL_FLUX_OPERATOR_CATEGORIES)


def test_weight_tensors_are_checked_before_the_native_boundary():
    """Every weight pointer handed to the C ABI comes from a tensor checked for device, dtype,
    shape and contiguity (the kernels read raw pointers; a strided, host-resident or wrong-shape
    weight must be refused with a clean error, not read)."""
    from flux_amd.runtime.native_smollm2 import _model_weight_tensors

    model = _smol_geometry_model()
    cpu = torch.device("cpu")
    tensors = _model_weight_tensors(model, cpu)
    assert len(tensors) == 3 + 6 * 2
    assert tensors[0].data_ptr() == tensors[1].data_ptr()  # tied LM head
    with pytest.raises(ValueError, match="embedding weight is on cpu, expected cuda:0"):
        _model_weight_tensors(model, torch.device("cuda", 0))
    layer = model.model.layers[1]
    original = layer.self_attn.o_proj.weight
    layer.self_attn.o_proj.weight = torch.nn.Parameter(original.detach().t().contiguous().t())
    assert not layer.self_attn.o_proj.weight.is_contiguous()
    with pytest.raises(ValueError, match="layer 1 o_proj weight must be contiguous"):
        _model_weight_tensors(model, cpu)
    layer.self_attn.o_proj.weight = original
    layer.mlp.down_proj.weight = torch.nn.Parameter(torch.zeros(576, 1535))
    with pytest.raises(ValueError, match=r"layer 1 down weight has shape \[576, 1535\], expected \[576, 1536\]"):
        _model_weight_tensors(model, cpu)
    layer.mlp.down_proj.weight = torch.nn.Parameter(torch.zeros(576, 1536, dtype=torch.float64))
    with pytest.raises(ValueError, match="layer 1 down weight has dtype torch.float64"):
        _model_weight_tensors(model, cpu)
