"""``import macmetalpy as cp`` on the MI355X: this name is the reference
package's import name; it resolves to macmetalpy_amd so that code written
against the reference runs unchanged."""
import sys as _sys

import macmetalpy_amd as _impl

_sys.modules[__name__] = _impl
