from . import functional
from .modules import *  # noqa: F401,F403
from .modules import __all__ as _modules_all
from .backbones import SparseResNet, SparseResNet21D

__all__ = ["functional", "SparseResNet", "SparseResNet21D"] + list(_modules_all)
