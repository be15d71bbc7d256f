"""Native runtimes (mirror of the reference's ``flux.runtime``)."""

from flux_amd.runtime.native_smollm2 import (
    NativeDecodeRuntimeMemory,
    NativePrefillRuntimeMemory,
    NativeSmolLM2Decode,
    NativeSmolLM2LayerDecode,
    NativeSmolLM2Prefill,
    native_smollm2_greedy_generate,
    native_smollm2_prefill_is_available,
    native_smollm2_runtime_is_available,
)

__all__ = [
    "NativeDecodeRuntimeMemory",
    "NativePrefillRuntimeMemory",
    "NativeSmolLM2Decode",
    "NativeSmolLM2LayerDecode",
    "NativeSmolLM2Prefill",
    "native_smollm2_greedy_generate",
    "native_smollm2_prefill_is_available",
    "native_smollm2_runtime_is_available",
]
