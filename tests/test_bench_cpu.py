"""CPU checks of bench.py's HBM traffic figure: the committed rocprofv3 --pmc summary
of the fused decode kernel was measured on the kernel source in the tree, and its
per-token model reproduces the launch traffic the summary records."""

from __future__ import annotations

import bench


def _fields() -> dict:
    fields = {}
    for line in open(bench.TRAFFIC_PROFILE).read().splitlines():
        key, sep, value = line.partition(":")
        if sep:
            fields[key.strip().strip("*`- ")] = value.strip().strip("*` ")
    return fields


def test_traffic_profile_matches_the_decode_source():
    # None means a sha256 in the summary is not its source's: re-run the counters after a change to the
    # fused kernel or to the runtime that allocates its exchange arena.
    assert bench.profiled_traffic(128, 8192) is not None


def test_traffic_model_reproduces_the_recorded_launch():
    launch = _fields()["traffic_launch"]
    steps = int(launch.split("steps=")[1].split()[0])
    context = int(launch.split("context=")[1].split()[0])
    measured = int(launch.split("->")[1])
    modelled = bench.profiled_traffic(steps, context)
    assert abs(modelled - measured) <= 1e-6 * measured


def test_traffic_model_is_not_applied_below_its_fitted_range():
    minimum = int(_fields()["traffic_model_min_attended"])
    assert bench.profiled_traffic(128, minimum - 2) is None
    assert bench.profiled_traffic(128, minimum - 1) is not None
