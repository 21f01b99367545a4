"""MoBA (Mixture of Block Attention) for AMD MI355X (gfx950).

The same Python API as ZuricZ/moba-triton's `moba` package (`MoBAConfig`,
`moba_attention`, the `kernels.*` launchers), backed by hand-written HIP
kernels in `libmoba_hip.so` behind a C ABI (`include/moba_hip.h`).
"""

from moba.config import MoBAConfig
from moba.kernels.attention import moba_attention

__all__ = ["MoBAConfig", "moba_attention"]
__version__ = "0.1.0"
