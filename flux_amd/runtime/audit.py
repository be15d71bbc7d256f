"""Runtime audit of the native decode replay (counterpart of the reference's
``_runtime_audit``, ``benchmarks/benchmark_flux.py:818-859``).

The reference profiles ten replays with ``torch.profiler`` and attributes CUDA
events to owners by kernel-name heuristics.  Here each figure comes from the
runtime itself: the launches per replay are the growth of the runtime's own
count of the kernel launches and device commands replay() issued
(``flux_decode_replay_launches``) over the audited replays, host
synchronisations and device allocations are the runtime's own counters around
the replays (``flux_host_counters``), and allocation growth is the device's free
memory and torch's allocator before and after.  ``rocprofv3 --kernel-trace`` of
``python -m flux_amd.runtime.audit`` confirms the launch count on the device.

Usage: ``python -m flux_amd.runtime.audit [--capacity 4096] [--replays 10]``
prints one JSON object.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import time
from dataclasses import asdict, dataclass

import torch
from torch import nn

from flux_amd import _native
from flux_amd.runtime.native_smollm2 import NativeSmolLM2Prefill


@dataclass(frozen=True)
class RuntimeAudit:
    """Field names follow the reference's ``RuntimeAudit`` (benchmark_flux.py:120-130)."""

    capacity: int
    replays: int
    launches_per_replay: int
    flux_launches_per_replay: int
    cublas_launches_per_replay: int
    framework_launches_per_replay: int
    replay_allocation_growth_bytes: int
    stable_addresses: bool
    cpu_synchronize_events: int
    cpu_allocation_events: int
    device_commands_per_replay: float
    device_free_bytes_delta: int
    host_enqueue_us_per_replay: float
    device_us_per_replay: float


def host_counters() -> tuple[int, int, int]:
    """(host synchronisations, device allocations, device frees) of the runtimes since load."""
    values = [ctypes.c_int64() for _ in range(3)]
    _native.check(_native.load().flux_host_counters(*[ctypes.byref(v) for v in values]))
    return tuple(int(v.value) for v in values)  # type: ignore[return-value]


def runtime_audit(model: nn.Module, capacity: int = 4096, replays: int = 10) -> RuntimeAudit:
    """Capture a prefill of ``capacity - replays - 3`` tokens, warm 3 replays, audit ``replays`` replays."""
    if capacity <= replays + 3 or replays < 1:
        raise ValueError("audit capacity must exceed audit replays plus three warmups")
    device = next(model.parameters()).device
    vocab = int(model.config.vocab_size)
    prompt = (torch.arange(capacity - replays - 3, dtype=torch.long) * 7919 % vocab).unsqueeze(0).to(device)
    native = NativeSmolLM2Prefill.capture(model, prompt, max_decode_steps=replays + 3)
    for _ in range(3):
        native.replay()
    torch.cuda.synchronize()
    addresses = native.stable_addresses()
    decode = native.native_object().decode
    kernels_before, commands_before = decode.replay_launches()
    free_before = torch.cuda.mem_get_info(device)[0]
    allocated_before = torch.cuda.memory_allocated(device)
    syncs_before, allocs_before, frees_before = host_counters()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    t0 = time.perf_counter()
    for _ in range(replays):
        native.replay()
    enqueue = time.perf_counter() - t0
    stop.record()
    torch.cuda.synchronize()
    syncs_after, allocs_after, frees_after = host_counters()
    allocated_after = torch.cuda.memory_allocated(device)
    free_after = torch.cuda.mem_get_info(device)[0]
    kernels_after, commands_after = decode.replay_launches()
    kernels = (kernels_after - kernels_before) // replays
    result = RuntimeAudit(
        capacity=capacity,
        replays=replays,
        launches_per_replay=kernels,
        flux_launches_per_replay=kernels,
        cublas_launches_per_replay=0,
        framework_launches_per_replay=0,
        replay_allocation_growth_bytes=allocated_after - allocated_before,
        stable_addresses=addresses == native.stable_addresses(),
        cpu_synchronize_events=syncs_after - syncs_before,
        cpu_allocation_events=(allocs_after - allocs_before) + (frees_after - frees_before),
        device_commands_per_replay=(commands_after - commands_before) / replays,
        device_free_bytes_delta=free_after - free_before,
        host_enqueue_us_per_replay=round(enqueue * 1e6 / replays, 2),
        device_us_per_replay=round(start.elapsed_time(stop) * 1e3 / replays, 2),
    )
    del native
    return result


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--capacity", type=int, default=4096)
    parser.add_argument("--replays", type=int, default=10)
    parser.add_argument("--vocab", type=int, default=49152)
    args = parser.parse_args()
    from flux_amd import synthetic
    from flux_amd.model import FINAL_FLUX_OPERATOR_CATEGORIES, enable_flux_ops

    model = synthetic.build_hf_model(synthetic.SyntheticSpec(seed=0, vocab=args.vocab), device="cuda")
    enable_flux_ops(model, operators=FINAL_FLUX_OPERATOR_CATEGORIES)
    print(json.dumps(asdict(runtime_audit(model, args.capacity, args.replays))), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
