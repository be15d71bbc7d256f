"""Shared fixtures.  ``-m gpu`` tests need an MI355X and the built library;
``-m "not gpu"`` tests run anywhere (CPU only)."""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and libflux_amd.so")


def golden(name: str) -> dict[str, np.ndarray]:
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as data:
        return {k: data[k] for k in data.files}


@pytest.fixture(scope="session")
def gpu_device() -> torch.device:
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no ROCm GPU is visible")
    from flux_amd import _native

    _native.load()  # fail loudly when the HIP library is missing
    return torch.device("cuda:0")


def _flux_model(seed: int, vocab: int, device: torch.device):
    from flux_amd import synthetic
    from flux_amd.model import FINAL_FLUX_OPERATOR_CATEGORIES, enable_flux_ops

    model = synthetic.build_hf_model(synthetic.SyntheticSpec(seed=seed, vocab=vocab), device=device)
    enable_flux_ops(model, operators=FINAL_FLUX_OPERATOR_CATEGORIES)
    return model


@pytest.fixture(scope="session")
def smol_model(gpu_device):
    """Synthetic SmolLM2-135M (seed 0, vocab 49152) with Flux ops enabled, on the GPU."""
    return _flux_model(0, 49152, gpu_device)


@pytest.fixture(scope="session")
def small_model(gpu_device):
    """Reference system-test geometry with vocab 128 (seed 2701), Flux ops enabled."""
    return _flux_model(2701, 128, gpu_device)
