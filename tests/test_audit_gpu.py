"""Runtime audit of the native decode replay (the reference's audit mode,
benchmarks/benchmark_flux.py:818-859): one kernel launch per replay, no
allocation growth, stable buffer addresses, no host synchronisation and no
device allocation inside steady replay."""

from __future__ import annotations

import gc

import pytest

from flux_amd.runtime.audit import host_counters, runtime_audit

pytestmark = pytest.mark.gpu


def test_decode_replay_audit(small_model):
    audit = runtime_audit(small_model, capacity=4096, replays=10)
    assert audit.launches_per_replay == 1 and audit.flux_launches_per_replay == 1
    # The replay is that one launch: no token copy, and no event wait between replays on
    # one stream.
    assert audit.device_commands_per_replay == 1
    assert audit.cublas_launches_per_replay == 0 and audit.framework_launches_per_replay == 0
    assert audit.replay_allocation_growth_bytes == 0 and audit.device_free_bytes_delta == 0
    assert audit.stable_addresses
    assert audit.cpu_synchronize_events == 0 and audit.cpu_allocation_events == 0
    # Replays are enqueued asynchronously: the host returns long before the device finishes.
    assert audit.host_enqueue_us_per_replay < audit.device_us_per_replay


def test_counters_see_runtime_construction(small_model):
    syncs, allocs, frees = host_counters()
    runtime_audit(small_model, capacity=64, replays=2)
    gc.collect()  # the runtime's tensor views hold it in reference cycles
    syncs2, allocs2, frees2 = host_counters()
    # Construction allocates and warms up (synchronising); destruction frees everything it allocated.
    assert allocs2 > allocs and syncs2 > syncs
    assert allocs2 - allocs == frees2 - frees
