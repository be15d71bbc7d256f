"""Model integration (mirror of the reference's ``flux.model``)."""

from flux_amd.model.smollm2_flux import (
    FINAL_FLUX_OPERATOR_CATEGORIES,
    FLUX_OPERATOR_CATEGORIES,
    enable_flux_ops,
    flux_operator_counts,
)

__all__ = [
    "FINAL_FLUX_OPERATOR_CATEGORIES",
    "FLUX_OPERATOR_CATEGORIES",
    "enable_flux_ops",
    "flux_operator_counts",
]
