"""RMSNorm with the reference's numerics (sleuth/forge/model/norm.py:34-50): fp32 math
(F.rms_norm on x.float() with the gain in fp32), cast back to x's dtype. The attention
module never calls it on the HIP path (q/k norms run inside the kernels); it is the
module's parameter holder and the eager/training path."""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-5):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))
        self._f32: tuple[int, torch.Tensor] | None = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return F.rms_norm(x.float(), (x.shape[-1],), self.weight.float(), self.eps).to(x.dtype)

    def weight_f32(self) -> torch.Tensor:
        """The gain as a contiguous fp32 tensor on the weight's device, cached until the
        parameter changes (its version counter moves) -- what the HIP kernels read."""
        w = self.weight
        key = (w.data_ptr(), w._version, w.device)
        if self._f32 is None or self._f32[0] != key:
            self._f32 = (key, w.detach().to(torch.float32).contiguous())
        return self._f32[1]
