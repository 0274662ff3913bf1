"""The reference's import name for this package: ``import sparsetriton`` is ``sparsetriton_amd``.

Code written against the reference (``from sparsetriton import SparseTensor, randn``,
``from sparsetriton.nn.functional import sparse_conv3d``,
``from sparsetriton.utils.hash import HashTable`` ...) runs unchanged on the HIP
implementation: every ``sparsetriton.<sub>`` module name resolves to the very module object
``sparsetriton_amd.<sub>`` (one set of classes, one config state, whichever name imported
them).  The module tree mirrors the reference's (``sparsetriton/...`` in the reference tree).
"""

import importlib
import importlib.abc
import importlib.util
import sys

_IMPL = "sparsetriton_amd"
_ALIAS = __name__


class _AliasFinder(importlib.abc.MetaPathFinder, importlib.abc.Loader):
    """Resolves ``sparsetriton.<sub>`` to the already-importable ``sparsetriton_amd.<sub>``."""

    def __init__(self):
        self._specs = {}

    def find_spec(self, fullname, path=None, target=None):
        if not fullname.startswith(_ALIAS + "."):
            return None
        impl = _IMPL + fullname[len(_ALIAS):]
        try:
            if importlib.util.find_spec(impl) is None:
                return None
        except ModuleNotFoundError:
            return None
        return importlib.util.spec_from_loader(fullname, self)

    def create_module(self, spec):
        # the implementation module itself, so both names share one module object
        module = importlib.import_module(_IMPL + spec.name[len(_ALIAS):])
        self._specs[module.__name__] = module.__spec__
        return module

    def exec_module(self, module):
        # already executed under its own name; the import machinery re-pointed __spec__ at the
        # alias spec, so give the module back its own
        module.__spec__ = self._specs.pop(module.__name__, module.__spec__)


if not any(isinstance(f, _AliasFinder) for f in sys.meta_path):
    sys.meta_path.insert(0, _AliasFinder())

_impl = importlib.import_module(_IMPL)
from sparsetriton_amd import *  # noqa: E402,F401,F403
from sparsetriton_amd import __all__, __version__  # noqa: E402,F401

# submodules already imported by the implementation package are attributes here too
for _name in ("config", "nn", "tensor", "utils"):
    _mod = importlib.import_module(f"{_ALIAS}.{_name}")
    globals()[_name] = _mod
del _name, _mod
