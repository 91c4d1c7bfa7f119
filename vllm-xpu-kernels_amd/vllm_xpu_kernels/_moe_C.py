"""Op namespace torch.ops._moe_C (registered by _mi355moe_torch.so)."""
from . import _ops  # noqa: F401
