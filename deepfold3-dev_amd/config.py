"""Kernel selection config with the reference's field names.

The reference selects Triton kernels per site with ``OptimConfig`` booleans read
at construction (``src/deepfold3/model/config.py:683-881``). This package has
exactly one implementation of each hot-path module, the HIP one, chosen by
``use_hip_pairformer``. The reference's other levers are accepted (so configs
and presets carry over) but select nothing here. A module built with
``use_hip_pairformer=False`` refuses by name at construction
(:class:`~.inference_guard.NotActive`) instead of silently running something else.
"""

from __future__ import annotations

from dataclasses import dataclass

from . import kernel_census
from .inference_guard import NotActive

OPTIM_PRESETS = ("none", "inference", "hip")


@dataclass
class OptimConfig:
    use_hip_pairformer: bool = True
    # Reference levers (config.py:725-772); accepted for compatibility, no effect here.
    use_fused_evo_attention: bool = False
    use_fused_pair_bias: bool = False
    use_fused_swiglu: bool = False
    use_fused_transition_pair: bool = False
    use_fused_transition_single: bool = False
    use_fused_ada_transition: bool = False
    use_fused_triangle_mul: bool = False
    use_cueq_triangle_mul: bool = False
    use_channel_major_triangle_mul: bool = False
    use_fused_ln_transpose: bool = False
    use_fused_msa_transition_inference: bool = False
    use_fused_dropout_add: bool = True
    use_torch_compile: bool = False
    pair_chunk_budget_bytes: int = 0
    use_gradient_checkpointing: bool = False

    @classmethod
    def hip(cls) -> OptimConfig:
        """The HIP kernels at every hot-path site."""
        return cls(use_hip_pairformer=True)

    @classmethod
    def inference(cls) -> OptimConfig:
        """The reference's inference preset name; here it is the HIP path."""
        return cls(
            use_hip_pairformer=True,
            use_fused_evo_attention=True,
            use_fused_pair_bias=True,
            use_fused_swiglu=True,
            use_channel_major_triangle_mul=True,
            use_fused_transition_pair=True,
        )

    @classmethod
    def none(cls) -> OptimConfig:
        """Stock PyTorch at every site: not provided by this package (modules refuse)."""
        return cls(use_hip_pairformer=False, use_fused_dropout_add=False)

    @classmethod
    def from_preset(cls, name: str) -> OptimConfig:
        return {"none": cls.none, "inference": cls.inference, "hip": cls.hip}[name]()


def require_hip(site: str, optim: OptimConfig | None) -> None:
    """Refuse construction of a hot-path module when the HIP path is switched off."""
    if optim is not None and not optim.use_hip_pairformer:
        raise NotActive(site, "use_hip_pairformer=False: this package implements only the HIP kernels")
    kernel_census.requested(site, "hip")
