"""luma_amd -- LUMA (Log-space Unbiased Momentum AdamW) optimizer step for MI355X.

Drop-in for ``luma_optimizer``: ``from luma_amd import LUMA``.  The step runs
in hand-written HIP kernels (gfx950) behind the C ABI of include/luma.h; see
``luma_amd.optimizer``.
"""

from luma_amd import functional  # noqa: F401  (registers torch.ops.luma_amd.luma_step)
from luma_amd.config import get_kernel_config
from luma_amd.optimizer import LUMA

__all__ = ["LUMA", "get_kernel_config"]
__version__ = "0.1.0"
