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
* ``ctx{N}.npz``        config 2: prompts of N tokens (128 / 512 / 1024 / 2048 / 4096 /
                        8192) and 128 greedy tokens (513 at 8192: config 5 reaches
                        position 8704).  Every step keeps the token, the top-2 margin
                        and the top-8 logits; the steps in ``probe_steps`` also keep
                        the top-64 and the 256-index probe.  K/V slices after the
                        prompt (layers 0/15/29 at four positions, every layer at the
                        last prompt position).
* ``teacher_config1.npz`` / ``teacher_ctx8192.npz``  teacher forcing: after the
                        config-1 (ctx-8192) prompt, a seeded token sequence that
                        changes at every step is fed one token at a time; per-step
                        probes, full logits at the first and last steps and around
                        the middle, and every layer's K/V rows at the fed positions.
* ``tail_ctx8192.npz``  config 5's last 32 positions with changing tokens: after the
                        8192-token prompt, 480 greedy steps, then 32 seeded teacher tokens
                        at positions 8672..8703; top-8 logits at every step, probes in the
                        window, full logits at its first and last steps and every layer's K/V
                        rows at its first, middle and last fed positions.
* ``permuted.npz``      free-running greedy stream of the untied permuted-head model
                        (``synthetic.PERMUTED_HEAD_SPEC``), whose token changes at
                        every step: 64 tokens with per-step probes and full logits
                        at the first, second and last steps.
* ``small128.npz``      the reference system test's geometry with vocab 128 and
                        ids ``(arange*11+3) % 128`` (``tests/test_system.py:318-353``),
                        with the full logits of every step and every layer's K/V
                        at the last prompt position.
* ``ops.npz``           HF ``apply_rotary_pos_emb`` and ``LlamaRMSNorm`` input/output.
* ``rope.npz``          HF ``rotary_emb`` cos/sin rows at selected positions.

Run from the repo root: ``python tests/golden/make_golden.py [name ...]`` (no
names: every fixture).
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


def greedy_with_probes(model, prompt: torch.Tensor, new_tokens: int, *, probe_steps=None, teacher=None,
                       full_logit_steps=(), kv_steps=(), free_steps=0):
    """Greedy (or teacher-forced) decode with HF, recording per-step probes and K/V slices.

    Step 0's logits come from the prompt; step s >= 1 feeds ``teacher[s-1-free_steps]``
    when a teacher sequence is given and s > free_steps, else the previous step's argmax
    (so ``free_steps`` greedy steps run before the teacher window).  ``probe_steps``
    (default: every step) get the top-64 and 256-index probe; every step gets the
    token, the margin and the top-8.  ``full_logit_steps`` keep the whole logit
    row; ``kv_steps`` keep every layer's K/V row written by that step's token.
    """
    steps = new_tokens if teacher is None else free_steps + len(teacher) + 1
    probe_steps = list(range(steps)) if probe_steps is None else [s for s in probe_steps if s < steps]
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
        kv["k_all_last"] = np.stack([layer.keys[0][:, length - 1].numpy() for layer in cache.layers])
        kv["v_all_last"] = np.stack([layer.values[0][:, length - 1].numpy() for layer in cache.layers])
        logits = out.logits[0, -1]
        tokens, probes, top8v, top8i, margins, full, kv_rows = [], [], [], [], [], [], []
        for step in range(steps):
            values, indices = torch.topk(logits.float(), 8)
            top8v.append(values.numpy().astype(np.float32))
            top8i.append(indices.numpy().astype(np.int64))
            margins.append(np.float32(values[0] - values[1]))
            if step in probe_steps:
                probes.append(step_probes(logits))
            if step in full_logit_steps:
                full.append(logits.numpy().astype(np.float32).copy())
            token = int(torch.argmax(logits))
            tokens.append(token)
            if step + 1 == steps:
                break
            fed = token if teacher is None or step < free_steps else int(teacher[step - free_steps])
            out = model(input_ids=torch.tensor([[fed]]), past_key_values=cache, use_cache=True,
                        logits_to_keep=1)
            cache = out.past_key_values
            logits = out.logits[0, -1]
            if step + 1 in kv_steps:
                pos = length + step
                kv_rows.append((np.stack([layer.keys[0][:, pos].numpy() for layer in cache.layers]),
                                np.stack([layer.values[0][:, pos].numpy() for layer in cache.layers])))
    record = {
        "prompt": prompt[0].numpy().astype(np.int64),
        "tokens": np.asarray(tokens, dtype=np.int64),
        "kv_positions": np.asarray(positions, dtype=np.int64),
        "probe_indices": PROBE,
        "probe_steps": np.asarray(probe_steps, dtype=np.int64),
        "margin": np.asarray(margins, dtype=np.float32),
        "top8_values": np.stack(top8v),
        "top8_indices": np.stack(top8i),
    }
    for key in ("top_values", "top_indices", "probe"):
        record[key] = np.stack([p[key] for p in probes])
    if teacher is not None:
        record["teacher"] = np.asarray(teacher, dtype=np.int64)
        record["free_steps"] = np.int64(free_steps)
    if full_logit_steps:
        record["full_logit_steps"] = np.asarray([s for s in full_logit_steps if s < steps], dtype=np.int64)
        record["full_logits"] = np.stack(full)
    if kv_steps:
        record["kv_steps"] = np.asarray([s for s in kv_steps if s < steps], dtype=np.int64)
        record["kv_step_k"] = np.stack([k for k, _ in kv_rows])
        record["kv_step_v"] = np.stack([v for _, v in kv_rows])
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


def teacher_tokens(seed: int, count: int, vocab: int = 49152) -> np.ndarray:
    """A seeded uniform token sequence with no two equal neighbours."""
    rng = np.random.Generator(np.random.PCG64(5_000_011 + seed))
    tokens = rng.integers(0, vocab, size=count, dtype=np.int64)
    for i in range(1, count):
        if tokens[i] == tokens[i - 1]:
            tokens[i] = (tokens[i] + 1) % vocab
    return tokens


CONTEXT_LENGTHS = (128, 512, 1024, 2048, 4096, 8192)
CONFIG2_STEPS = 128
CONFIG5_STEPS = 513  # 8192-token prompt + 512 decode steps: positions 8192..8703


def main(selected: set[str]) -> None:
    torch.set_num_threads(os.cpu_count() or 1)
    want = (lambda name: not selected or name in selected)
    meta_path = os.path.join(OUT, "weights.json")
    meta: dict[str, object] = {}
    if os.path.exists(meta_path):
        with open(meta_path) as handle:
            meta = json.load(handle)
    meta.update({"transformers": __import__("transformers").__version__, "torch": torch.__version__,
                 "numpy": np.__version__})

    spec = synthetic.SyntheticSpec(seed=0)
    model = synthetic.build_hf_model(spec)
    meta["weights_seed0_vocab49152"] = synthetic.weights_sha256(synthetic.synthetic_state_dict(spec))
    if want("rope"):
        np.savez_compressed(os.path.join(OUT, "rope.npz"), **rope_fixture(model))
    if want("ops"):
        np.savez_compressed(os.path.join(OUT, "ops.npz"), **ops_fixture(model))

    if want("config1"):
        t = time.time()
        prompt = synthetic.synthetic_prompt(1, 128)
        record = greedy_with_probes(model, prompt, 32)
        check_against_generate(model, prompt, record["tokens"])
        np.savez_compressed(os.path.join(OUT, "config1.npz"), **record)
        print(f"config1 done in {time.time() - t:.1f}s tokens={record['tokens'][:8]}", flush=True)

    if want("teacher_config1"):
        t = time.time()
        prompt = synthetic.synthetic_prompt(1, 128)
        teacher = teacher_tokens(1, 48)
        record = greedy_with_probes(model, prompt, 0, teacher=teacher, full_logit_steps=(0, 1, 24, 48),
                                    kv_steps=(1, 2, 24, 48))
        np.savez_compressed(os.path.join(OUT, "teacher_config1.npz"), **record)
        print(f"teacher_config1 done in {time.time() - t:.1f}s argmax={record['tokens'][:8]}", flush=True)

    for length in CONTEXT_LENGTHS:
        name = f"ctx{length}"
        if not want(name) and not (length == 8192 and (want("teacher_ctx8192") or want("tail_ctx8192"))):
            continue
        prompt = synthetic.synthetic_prompt(2, length)
        if want(name):
            t = time.time()
            steps = CONFIG5_STEPS if length == 8192 else CONFIG2_STEPS
            probe_steps = (0, 1, 2, 3, 31, 63, 127) + ((255, 511, 512) if length == 8192 else ())
            record = greedy_with_probes(model, prompt, steps, probe_steps=probe_steps)
            np.savez_compressed(os.path.join(OUT, f"{name}.npz"), **record)
            print(f"{name} done in {time.time() - t:.1f}s tokens={sorted(set(record['tokens'].tolist()))} "
                  f"min margin={record['margin'].min():.4f}", flush=True)
        if length == 8192 and want("tail_ctx8192"):
            # Config 5's last 32 positions (8672..8703) with changing tokens: 480 greedy steps
            # after the 8192-token prompt, then 32 teacher-forced ones.
            t = time.time()
            teacher = teacher_tokens(3, 32)
            free = CONFIG5_STEPS - 1 - len(teacher)
            record = greedy_with_probes(model, prompt, 0, teacher=teacher, free_steps=free,
                                        probe_steps=(free, free + 1, free + 16, free + 32),
                                        full_logit_steps=(free + 1, free + 32),
                                        kv_steps=(free + 1, free + 16, free + 32))
            np.savez_compressed(os.path.join(OUT, "tail_ctx8192.npz"), **record)
            print(f"tail_ctx8192 done in {time.time() - t:.1f}s", flush=True)
        if length == 8192 and want("teacher_ctx8192"):
            t = time.time()
            teacher = teacher_tokens(2, 32)
            record = greedy_with_probes(model, prompt, 0, teacher=teacher, full_logit_steps=(0, 1, 32),
                                        kv_steps=(1, 32))
            np.savez_compressed(os.path.join(OUT, "teacher_ctx8192.npz"), **record)
            print(f"teacher_ctx8192 done in {time.time() - t:.1f}s", flush=True)

    if want("permuted"):
        t = time.time()
        pspec = synthetic.PERMUTED_HEAD_SPEC
        pmodel = synthetic.build_hf_model(pspec)
        meta["weights_permuted_head"] = synthetic.weights_sha256(synthetic.synthetic_state_dict(pspec))
        prompt = synthetic.synthetic_prompt(1, 128)
        record = greedy_with_probes(pmodel, prompt, 64, full_logit_steps=(0, 1, 63))
        check_against_generate(pmodel, prompt, record["tokens"])
        tokens = record["tokens"].tolist()
        assert all(a != b for a, b in zip(tokens, tokens[1:])), "permuted-head stream repeats a token"
        np.savez_compressed(os.path.join(OUT, "permuted.npz"), **record)
        print(f"permuted done in {time.time() - t:.1f}s tokens={tokens[:8]} min margin={record['margin'].min():.3f}",
              flush=True)

    if want("small128"):
        small = synthetic.SyntheticSpec(seed=2701, vocab=128)
        small_model = synthetic.build_hf_model(small)
        meta["weights_seed2701_vocab128"] = synthetic.weights_sha256(synthetic.synthetic_state_dict(small))
        prompt = (torch.arange(7).unsqueeze(0) * 11 + 3) % 128
        record = greedy_with_probes(small_model, prompt, 8, full_logit_steps=tuple(range(8)))
        check_against_generate(small_model, prompt, record["tokens"])
        prompt17 = (torch.arange(17).unsqueeze(0) * 11 + 3) % 128
        record17 = greedy_with_probes(small_model, prompt17, 4, full_logit_steps=tuple(range(4)))
        record.update({f"p17_{k}": v for k, v in record17.items()})
        np.savez_compressed(os.path.join(OUT, "small128.npz"), **record)

    with open(meta_path, "w") as handle:
        json.dump(meta, handle, indent=2, sort_keys=True)
    print("golden vectors written", flush=True)


if __name__ == "__main__":
    main(set(sys.argv[1:]))
