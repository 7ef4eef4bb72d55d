"""IR -> gfx950 HIP lowering (counterpart of ``warpir/lowering/__init__.py:1-5``).

The reference exports ``ThunderKittensLowerer`` (H100 CUDA).  This target
exports ``CDNA4Lowerer`` with the same ``lower(kernel) -> str`` method.
"""
from .cdna4 import CDNA4Lowerer, CDNA4Target, LaunchConfig, LoweringError

__all__ = ["CDNA4Lowerer", "CDNA4Target", "LaunchConfig", "LoweringError"]
