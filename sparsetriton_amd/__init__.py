"""MI355X-native sparse 3-D convolution with the sparsetriton Python API.

``SparseTensor``, ``randn``, ``nn.SubMConv3D`` / ``SparseConv3D`` /
``SparseConvTransposed3D``, ``nn.functional.sparse_conv3d`` and
``config.set_conv_algo`` behave as in the reference package; the coordinate
hash, kernel maps and gather-GEMM forward / backward run as hand-written HIP
kernels for gfx950 in ``libsparsetriton_amd.so`` (C ABI in
``include/sparsetriton_amd.h``).
"""

from . import config
from .config import ConvAlgo, get_conv_algo, set_conv_algo
from .tensor import SparseTensor, TensorCache, randn
from . import nn

__all__ = ["SparseTensor", "TensorCache", "randn", "nn", "config", "ConvAlgo", "set_conv_algo", "get_conv_algo"]
__version__ = "0.1.0"
