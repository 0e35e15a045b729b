"""fastmlx_amd -- MI355X-native quantized linear path (MLX affine quantization).

The compute lives in ``libfmxq.so`` (hand-written HIP for gfx950); this package
binds it.  ``ops`` exposes the raw kernel ABI over torch device tensors.
"""
from ._lib import FmxqError, load  # noqa: F401

__all__ = ["FmxqError", "load"]
