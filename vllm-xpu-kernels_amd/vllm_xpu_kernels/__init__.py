"""MI355X (gfx950) fused Mixture-of-Experts kernels behind the
vllm-xpu-kernels op surface (torch.ops._moe_C / _C / _xpu_C and
fused_moe_interface.XpuFusedMoe)."""
from . import _ops  # noqa: F401  (loads the HIP library; raises if missing)

__all__ = ["fused_moe_interface", "ops"]
