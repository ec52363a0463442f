"""``import macmetalpy as cp`` on the MI355X: this name is the reference
package's import name; it resolves to macmetalpy_amd so that code written
against the reference runs unchanged.  Submodule imports
(``from macmetalpy._kernel_cache import KernelCache``) resolve to the same
module objects of macmetalpy_amd, never to second copies."""
import importlib as _importlib
import importlib.abc as _abc
import importlib.util as _util
import sys as _sys

import macmetalpy_amd as _impl

_PREFIX = __name__ + "."


class _SubmoduleAlias(_abc.MetaPathFinder, _abc.Loader):
    """Maps ``macmetalpy.X`` to the already-importable ``macmetalpy_amd.X``."""

    def find_spec(self, fullname, path=None, target=None):
        if not fullname.startswith(_PREFIX):
            return None
        real = "macmetalpy_amd." + fullname[len(_PREFIX):]
        if _util.find_spec(real) is None:
            return None
        return _util.spec_from_loader(fullname, self, origin=real)

    def create_module(self, spec):
        return _importlib.import_module(spec.origin)

    def exec_module(self, module):
        pass


if not any(isinstance(f, _SubmoduleAlias) for f in _sys.meta_path):
    _sys.meta_path.insert(0, _SubmoduleAlias())
_sys.modules[__name__] = _impl
