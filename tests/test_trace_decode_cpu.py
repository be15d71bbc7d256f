"""CPU checks of ``flux_amd.trace_decode``'s table (no GPU: the trace buffers are faked)."""

from __future__ import annotations

import ctypes

import numpy as np

from flux_amd import trace_decode


class _FakeTraceLibrary:
    """Fills the four trace buffers the way the FLUX_TRACE kernel lays them out."""

    def __init__(self) -> None:
        phases = np.zeros((512, 16), dtype=np.uint64)
        # 256 workgroups; workgroup w reaches slot s at tick 1000 + 100 * s + w (1 tick = 10 ns).
        for slot in range(13):
            phases[:256, slot] = 1000 + 100 * slot + np.arange(256)
        phases[36:, 5] = 0  # only the 36 merge workgroups record slot 5
        attention = np.zeros((512, 8), dtype=np.uint64)
        attention[:255, :4] = 2000
        attention[:36, 4:6] = 3000
        copies = np.zeros((256, 8, 4), dtype=np.uint64)
        copies[:255, :, :] = 1500
        per_layer = np.zeros((4, 31, 16), dtype=np.uint64)
        per_layer[0, :, 0] = 1000 + 1450 * np.arange(31)  # 14.5 us layers
        # Final phase (row 30) of the four traced workgroups: start, h fetched, argmax, token.
        per_layer[:, 30, 0] = 1000 + 1450 * 30
        per_layer[:, 30, 1] = 1000 + 1450 * 30 + 160 + np.arange(4)
        per_layer[:, 30, 2] = 1000 + 1450 * 30 + 1800
        per_layer[:, 30, 3] = 1000 + 1450 * 30 + 2100
        self.buffers = {
            "flux_debug_trace_all": phases,
            "flux_debug_attn_trace": attention,
            "flux_debug_copy_trace": copies,
            "flux_debug_trace": per_layer,
        }

    def __getattr__(self, name: str):
        source = self.buffers[name]

        def read(pointer: ctypes.c_void_p) -> int:
            ctypes.memmove(pointer.value, source.ctypes.data, source.nbytes)
            return 0

        return read


def _row(lines: list[str], label: str) -> list[str]:
    [row] = [line for line in lines if line.startswith(f"| {label} |")]
    return [cell.strip() for cell in row.strip("|").split("|")]


def test_trace_table_times_are_relative_to_the_first_phase_a_start():
    lines = trace_decode.trace_launch(_FakeTraceLibrary())
    # Slot 0 starts at tick 1000 for workgroup 0 and 1255 for workgroup 255.
    assert _row(lines, "A start (QKV rows)") == ["A start (QKV rows)", "1.27", "2.55", "0.00", "256"]
    # Slot 12 (gate/up published) is listed under its own name, 12 * 100 ticks = 12 us later.
    assert _row(lines, "D gate/up published")[3] == "12.00"
    # Only workgroups that record a point are counted.
    assert _row(lines, "B2 partials fetched (merge WGs)")[4] == "36"
    assert _row(lines, "attention QK^T done") == ["attention QK^T done", "10.00", "10.00", "10.00", "255"]
    assert _row(lines, "merge global max done")[1:] == ["20.00", "20.00", "20.00", "36"]
    assert _row(lines, "K/V copy landed, wave 7")[1:] == ["5.00", "5.00", "5.00", "255"]
    [durations] = [line for line in lines if line.startswith("workgroup 0, layer durations")]
    assert durations.endswith(" ".join(["14.50"] * 30))
    assert lines[-3].startswith("LM head phase, final h fetched: 1.60 1.61 1.62 1.63 us")
    assert lines[-1].startswith("LM head phase, token chosen: 21.00 21.00 21.00 21.00 us")


def test_trace_buffers_match_the_kernel_declarations():
    import pathlib

    source = (pathlib.Path(trace_decode.__file__).parent / "csrc" / "decode_kernels.hip").read_text()
    assert "g_flux_trace[4][kLayers + 1][16]" in source
    assert "g_flux_trace_all[512][16]" in source
    assert "g_flux_attn_trace[512][8]" in source
    assert "g_flux_copy_trace[256][8][4]" in source
