"""Write the golden vectors for the SmolLM2 FP32 token loop.

The reference FP32 path that Flux validates against is Hugging Face
``LlamaForCausalLM`` eager FP32 (``/root/reference/tests/test_system.py:356-497``,
``flux/model/smollm2.py:27-33``); the reference commits no fixtures of its own.
This script runs the *third-party* transformers package (5.15.0 in the build
image) on the CPU -- never the reference's code -- with the repo's seeded
synthetic weights, and stores small vectors under ``tests/golden/``:

* ``weights.json``      SHA-256 of the synthetic weights (seed 0 / vocab 49152, and
                        seed 2701 / vocab 128) and of the RoPE tables.
* ``config1.npz``       config 1: 128-token prompt, 32 greedy tokens, per-step
                        top-64 logits, a fixed 256-index logit probe, top-2 margins,
                        and K/V slices after the prompt.
* ``ctx{N}.npz``        prompts of N tokens (512 / 1024 / 2048 / 8192), greedy
                        continuation with the same per-step probes.
* ``small128.npz``      the reference system test's geometry with vocab 128 and
                        ids ``(arange*11+3) % 128`` (``tests/test_system.py:318-353``).
* ``ops.npz``           HF ``apply_rotary_pos_emb`` and ``LlamaRMSNorm`` input/output.
* ``rope.npz``          HF ``rotary_emb`` cos/sin rows at selected positions.

Run from the repo root: ``python tests/golden/make_golden.py``.
"""

from __future__ import annotations

import hashlib
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from flux_amd import synthetic  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
PROBE = np.random.Generator(np.random.PCG64(77)).choice(49152, size=256, replace=False).astype(np.int64)
KV_LAYERS = (0, 15, 29)
KV_POSITIONS_FRACTION = (0.0, 0.25, 0.5, 1.0)


def step_probes(logits: torch.Tensor, top: int = 64) -> dict[str, np.ndarray]:
    values, indices = torch.topk(logits.float(), top)
    return {
        "top_values": values.numpy().astype(np.float32),
        "top_indices": indices.numpy().astype(np.int64),
        "probe": logits[torch.from_numpy(PROBE[PROBE < logits.numel()])].numpy().astype(np.float32),
        "margin": np.float32(values[0] - values[1]),
    }


def greedy_with_probes(model, prompt: torch.Tensor, new_tokens: int):
    """Greedy decode with HF, recording per-step probes and K/V slices after the prompt."""
    with torch.inference_mode():
        out = model(input_ids=prompt, use_cache=True, logits_to_keep=1)
        cache = out.past_key_values
        length = prompt.shape[1]
        positions = sorted({min(length - 1, int(f * (length - 1))) for f in KV_POSITIONS_FRACTION})
        kv = {}
        for layer in KV_LAYERS:
            if layer < len(cache.layers):
                kv[f"k{layer}"] = cache.layers[layer].keys[0][:, positions].numpy().copy()
                kv[f"v{layer}"] = cache.layers[layer].values[0][:, positions].numpy().copy()
        logits = out.logits[0, -1]
        tokens, probes = [], []
        for step in range(new_tokens):
            probes.append(step_probes(logits))
            token = int(torch.argmax(logits))
            tokens.append(token)
            if step + 1 == new_tokens:
                break
            out = model(input_ids=torch.tensor([[token]]), past_key_values=cache, use_cache=True,
                        logits_to_keep=1)
            cache = out.past_key_values
            logits = out.logits[0, -1]
    record = {
        "prompt": prompt[0].numpy().astype(np.int64),
        "tokens": np.asarray(tokens, dtype=np.int64),
        "kv_positions": np.asarray(positions, dtype=np.int64),
        "probe_indices": PROBE,
    }
    for key in ("top_values", "top_indices", "probe", "margin"):
        record[key] = np.stack([p[key] for p in probes])
    record.update(kv)
    return record


def check_against_generate(model, prompt: torch.Tensor, tokens: np.ndarray) -> None:
    with torch.inference_mode():
        expected = model.generate(input_ids=prompt, do_sample=False, num_beams=1,
                                  max_new_tokens=len(tokens), use_cache=True, pad_token_id=0)
    assert expected[0, prompt.shape[1]:].numpy().tolist() == tokens.tolist(), "generate() disagrees"


def rope_fixture(model) -> dict[str, np.ndarray]:
    rows = np.asarray([0, 1, 2, 127, 1000, 4095, 8191, 8192, 8703], dtype=np.int64)
    positions = torch.arange(8704).unsqueeze(0)
    seed = model.model.embed_tokens.weight[:1].view(1, 1, 576)
    with torch.inference_mode():
        cos, sin = model.model.rotary_emb(seed, positions)
    cos = cos.reshape(8704, 64).contiguous()
    sin = sin.reshape(8704, 64).contiguous()
    return {
        "rows": rows,
        "cos": cos[rows].numpy(),
        "sin": sin[rows].numpy(),
        "cos_sha256": np.frombuffer(hashlib.sha256(cos.numpy().tobytes()).digest(), dtype=np.uint8),
        "sin_sha256": np.frombuffer(hashlib.sha256(sin.numpy().tobytes()).digest(), dtype=np.uint8),
    }


def ops_fixture(model) -> dict[str, np.ndarray]:
    from transformers.models.llama.modeling_llama import LlamaRMSNorm, apply_rotary_pos_emb

    g = torch.Generator().manual_seed(1307)
    q = torch.randn(1, 9, 5, 64, generator=g)
    k = torch.randn(1, 3, 5, 64, generator=g)
    positions = torch.tensor([[0, 1, 17, 4096, 8191]])
    with torch.inference_mode():
        cos, sin = model.model.rotary_emb(q, positions)
        q_embed, k_embed = apply_rotary_pos_emb(q, k, cos, sin)
    norm = LlamaRMSNorm(576, eps=1e-5)
    x = torch.randn(4, 576, generator=g)
    with torch.no_grad():
        norm.weight.copy_(torch.randn(576, generator=g))
        y = norm(x)
    return {
        "rope_q": q.numpy(), "rope_k": k.numpy(), "rope_positions": positions.numpy(),
        "rope_cos": cos.numpy(), "rope_sin": sin.numpy(),
        "rope_q_embed": q_embed.numpy(), "rope_k_embed": k_embed.numpy(),
        "norm_x": x.numpy(), "norm_w": norm.weight.detach().numpy(), "norm_y": y.detach().numpy(),
    }


def main() -> None:
    torch.set_num_threads(os.cpu_count() or 1)
    meta: dict[str, object] = {"transformers": __import__("transformers").__version__,
                               "torch": torch.__version__, "numpy": np.__version__}

    spec = synthetic.SyntheticSpec(seed=0)
    model = synthetic.build_hf_model(spec)
    meta["weights_seed0_vocab49152"] = synthetic.weights_sha256(synthetic.synthetic_state_dict(spec))
    np.savez_compressed(os.path.join(OUT, "rope.npz"), **rope_fixture(model))
    np.savez_compressed(os.path.join(OUT, "ops.npz"), **ops_fixture(model))

    t = time.time()
    prompt = synthetic.synthetic_prompt(1, 128)
    record = greedy_with_probes(model, prompt, 32)
    check_against_generate(model, prompt, record["tokens"])
    np.savez_compressed(os.path.join(OUT, "config1.npz"), **record)
    print(f"config1 done in {time.time() - t:.1f}s tokens={record['tokens'][:8]}", flush=True)

    for length, steps in ((512, 8), (1024, 8), (2048, 8), (8192, 4)):
        t = time.time()
        prompt = synthetic.synthetic_prompt(2, length)
        record = greedy_with_probes(model, prompt, steps)
        np.savez_compressed(os.path.join(OUT, f"ctx{length}.npz"), **record)
        print(f"ctx{length} done in {time.time() - t:.1f}s margins={record['margin']}", flush=True)

    small = synthetic.SyntheticSpec(seed=2701, vocab=128)
    small_model = synthetic.build_hf_model(small)
    meta["weights_seed2701_vocab128"] = synthetic.weights_sha256(synthetic.synthetic_state_dict(small))
    prompt = (torch.arange(7).unsqueeze(0) * 11 + 3) % 128
    record = greedy_with_probes(small_model, prompt, 8)
    check_against_generate(small_model, prompt, record["tokens"])
    prompt17 = (torch.arange(17).unsqueeze(0) * 11 + 3) % 128
    record17 = greedy_with_probes(small_model, prompt17, 4)
    record.update({f"p17_{k}": v for k, v in record17.items()})
    np.savez_compressed(os.path.join(OUT, "small128.npz"), **record)

    with open(os.path.join(OUT, "weights.json"), "w") as handle:
        json.dump(meta, handle, indent=2, sort_keys=True)
    print("golden vectors written", flush=True)


if __name__ == "__main__":
    main()
