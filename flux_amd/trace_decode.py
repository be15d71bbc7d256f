"""Phase timeline of one layer of the fused decode kernel (diagnostic tool).

Runs the token loop of ``libflux_amd_trace.so`` (the ``FLUX_TRACE`` build made by
``python -m flux_amd.build --trace``) on a synthetic SmolLM2-135M model and prints,
for layer 15 of the third token of each launch, when each phase point was reached,
in microseconds after the earliest phase-A start over all workgroups (median, max
and min over the workgroups that pass the point).  Usage on a GPU host::

    python -m flux_amd.trace_decode [--context 8192] [--launches 3]

The timestamps come from the device wall clock (``wall_clock64``, 100 MHz).  The
trace build writes them from one lane per workgroup (per wave for the K/V copy
points), so the traced launch runs a few stores slower than the normal library,
which has none of them.
"""

from __future__ import annotations

import argparse
import ctypes
import os

import numpy as np
import torch

from flux_amd import _native, synthetic
from flux_amd.build import TRACE_LIBRARY

TICKS_PER_US = 100.0

# Slots of the per-workgroup phase trace, in the order the kernel reaches them.
PHASE_POINTS = (
    (0, "A start (QKV rows)"),
    (1, "A input vector fetched"),
    (2, "B start (A published)"),
    (3, "B query and K/V staged"),
    (4, "B partials published"),
    (5, "B2 partials fetched (merge WGs)"),
    (6, "C start (B2 published)"),
    (7, "C merged heads fetched"),
    (8, "D start (C published)"),
    (9, "D normed vector fetched"),
    (12, "D gate/up published"),
    (10, "E start"),
    (11, "E activations fetched"),
)
ATTENTION_POINTS = (
    (0, "attention QK^T done"),
    (1, "attention softmax done"),
    (2, "attention PV done"),
    (3, "attention partial stored"),
    (4, "merge global max done"),
    (5, "merge sums in LDS"),
)
COPY_POINTS = (
    (3, "K/V copy start"),
    (0, "K/V copy issued"),
    (1, "query poll done"),
    (2, "K/V copy landed"),
)


def _read(lib: ctypes.CDLL, name: str, shape: tuple[int, ...]) -> np.ndarray:
    out = np.zeros(shape, dtype=np.uint64)
    status = getattr(lib, name)(out.ctypes.data_as(ctypes.c_void_p))
    if status != 0:
        raise RuntimeError(f"{name} returned HIP status {status}")
    return out.astype(np.int64)


def _row(label: str, ticks: np.ndarray, t0: int) -> str:
    ticks = ticks[ticks > 0]
    if ticks.size == 0:
        return f"| {label} | - | - | - | 0 |"
    us = (ticks - t0) / TICKS_PER_US
    return f"| {label} | {np.median(us):.2f} | {us.max():.2f} | {us.min():.2f} | {ticks.size} |"


def trace_launch(lib: ctypes.CDLL) -> list[str]:
    """Format the timeline the last launch left in the trace buffers."""
    phases = _read(lib, "flux_debug_trace_all", (512, 16))
    attention = _read(lib, "flux_debug_attn_trace", (512, 8))
    copies = _read(lib, "flux_debug_copy_trace", (256, 8, 4))
    per_layer = _read(lib, "flux_debug_trace", (4, 31, 16))
    starts = phases[:, 0]
    t0 = int(starts[starts > 0].min())
    lines = ["| point | median us | max us | min us | WGs |", "|---|---:|---:|---:|---:|"]
    lines += [_row(name, phases[:, slot], t0) for slot, name in PHASE_POINTS]
    lines += [_row(name, attention[:, slot], t0) for slot, name in ATTENTION_POINTS]
    for slot, name in COPY_POINTS:
        for wave in (0, 7):
            lines.append(_row(f"{name}, wave {wave}", copies[:, wave, slot], t0))
    layer_starts = per_layer[0, :, 0]
    durations = np.diff(layer_starts[:31]) / TICKS_PER_US
    lines.append("")
    lines.append("workgroup 0, layer durations (us, layers 0-29): " + " ".join(f"{d:.2f}" for d in durations))
    # The final phase (slot row 30): start, final-norm input fetched with the first LM-head
    # rows requested, the workgroup's argmax done, the token chosen from every workgroup's.
    lm = per_layer[:, 30, :4]
    start = int(lm[:, 0][lm[:, 0] > 0].min())
    for name, slot in (("final h fetched", 1), ("workgroup argmax", 2), ("token chosen", 3)):
        us = (lm[:, slot][lm[:, slot] > 0] - start) / TICKS_PER_US
        lines.append(f"LM head phase, {name}: " + " ".join(f"{u:.2f}" for u in us) +
                     " us after its start (workgroups 0, 85, 170, 255)")
    return lines


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--context", type=int, default=8192, help="prompt length before the traced tokens")
    parser.add_argument("--launches", type=int, default=3, help="traced token-loop launches")
    args = parser.parse_args()
    if not os.path.exists(TRACE_LIBRARY):
        raise SystemExit(f"{TRACE_LIBRARY} is missing: run `python -m flux_amd.build --trace` first")
    lib = _native.load(TRACE_LIBRARY)
    # Imported after the traced library is loaded so every native call binds to it.
    from flux_amd.model import FINAL_FLUX_OPERATOR_CATEGORIES, enable_flux_ops
    from flux_amd.runtime import NativeSmolLM2Prefill

    device = torch.device("cuda:0")
    model = synthetic.build_hf_model(synthetic.SyntheticSpec(seed=0), device=device)
    enable_flux_ops(model, operators=FINAL_FLUX_OPERATOR_CATEGORIES)
    prompt = synthetic.synthetic_prompt(2, args.context).to(device)
    runtime = NativeSmolLM2Prefill.capture(model, prompt, max_decode_steps=64)
    for launch in range(args.launches):
        runtime.prefill(prompt)
        torch.cuda.synchronize()
        runtime.native_object().decode.generate_greedy(8)
        torch.cuda.synchronize()
        print(f"launch {launch}, context {args.context}: layer 15 of token 2, "
              "us after the earliest phase-A start", flush=True)
        print("\n".join(trace_launch(lib)), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
