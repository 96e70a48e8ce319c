"""MI355X (gfx950) native N-dimensional dense convolution with the torch-convnd API.

Importing defines the ``torch_convnd`` operator schemas but loads no native code; the
gfx950 libraries load on the first native call (or ``load_native()``).
"""

from ._build import load_native
from ._dispatch import ensure_compatible_operator
from ._operators import ensure_native_definitions
from ._version import __version__
from .diagnostics import get_runtime_info
from .functional import conv_nd
from .modules import (
    Conv1d,
    Conv2d,
    Conv3d,
    Conv4d,
    ConvNd,
    PartialConv1d,
    PartialConv2d,
    PartialConv3d,
    PartialConv4d,
    PartialConvNd,
    PartialSequential,
)
from .partial import PartialConvOutput, partial_conv_nd

ensure_native_definitions()
ensure_compatible_operator()

__all__ = [
    "Conv1d",
    "Conv2d",
    "Conv3d",
    "Conv4d",
    "ConvNd",
    "PartialConv1d",
    "PartialConv2d",
    "PartialConv3d",
    "PartialConv4d",
    "PartialConvNd",
    "PartialConvOutput",
    "PartialSequential",
    "conv_nd",
    "partial_conv_nd",
    "load_native",
    "get_runtime_info",
    "__version__",
]
