"""flux_amd: MI355X-native (gfx950 HIP) SmolLM2 FP32 batch-1 token loop.

Mirrors the reference's public surface:
``flux_amd.model.enable_flux_ops`` (``flux.model``) and
``flux_amd.runtime.{NativeSmolLM2Prefill, NativeSmolLM2Decode,
native_smollm2_greedy_generate}`` (``flux.runtime``).  The native code is
``flux_amd/lib/libflux_amd.so`` (C ABI ``include/flux_amd.h``), built by
``python -m flux_amd.build``.
"""

__version__ = "0.1.0"
