"""RMSNorm module backed by the gfx950 norm kernel (K6).

Drop-in for transformers' ``Qwen3MoeRMSNorm`` (tf:284-302, forward
tf:294-299): an ``nn.Module`` with the same ``weight`` parameter and
``variance_epsilon``, computing bf16(weight * bf16(x * rsqrt(mean(x^2) +
eps))) in one kernel instead of the eager module's seven or eight.  The
fp32 sum of squares runs in the kernel's own order, so outputs may differ
from the eager module by a last-place rounding of the variance.
"""
from __future__ import annotations

import torch
from torch import nn

from .. import ops


class Qwen3RMSNormHip(nn.Module):
    def __init__(self, weight: nn.Parameter, eps: float) -> None:
        super().__init__()
        self.weight = weight
        self.variance_epsilon = float(eps)

    @classmethod
    def from_module(cls, norm: nn.Module) -> "Qwen3RMSNormHip":
        """Wrap an HF ``Qwen3MoeRMSNorm`` (shares its weight parameter)."""
        return cls(norm.weight, norm.variance_epsilon)

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        if hidden_states.dtype != torch.bfloat16 or self.weight.dtype != torch.bfloat16:
            raise ValueError("Qwen3RMSNormHip computes bf16 activations with a bf16 weight")
        return ops.rms_norm(hidden_states, self.weight, self.variance_epsilon)

    def extra_repr(self) -> str:
        return f"{tuple(self.weight.shape)}, eps={self.variance_epsilon}"


def install_hip_norms(model: nn.Module) -> int:
    """Replace every ``Qwen3MoeRMSNorm`` submodule of ``model`` with a
    ``Qwen3RMSNormHip`` sharing its weight; returns how many were replaced."""
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeRMSNorm

    targets = [(name, mod) for name, mod in model.named_modules()
               if isinstance(mod, Qwen3MoeRMSNorm)]
    for name, mod in targets:
        parent_name, _, attr = name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        setattr(parent, attr, Qwen3RMSNormHip.from_module(mod))
    return len(targets)
