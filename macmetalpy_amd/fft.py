"""``cp.fft``: the real-valued helpers on the device; the transforms raise.

The reference's fft.py runs NumPy's FFT on the host and returns complex64
arrays that it keeps host-resident.  Device arrays here hold no complex
dtype, so the transforms (fft, ifft, rfft, ... hfft) raise
NotImplementedError instead of computing on the host.  fftfreq,
rfftfreq, fftshift and ifftshift produce real results and run on the
device with NumPy's definitions.
"""
from __future__ import annotations

import numpy as np

__all__ = ["fft", "ifft", "fft2", "ifft2", "fftn", "ifftn", "rfft", "irfft", "rfft2", "irfft2",
           "rfftn", "irfftn", "hfft", "ihfft", "fftfreq", "rfftfreq", "fftshift", "ifftshift"]


def _no_complex(name):
    def transform(*args, **kwargs):
        raise NotImplementedError(f"fft.{name} returns complex values; the device library holds "
                                  "no complex dtype")
    transform.__name__ = name
    return transform


for _name in ("fft", "ifft", "fft2", "ifft2", "fftn", "ifftn", "rfft", "irfft", "rfft2", "irfft2",
              "rfftn", "irfftn", "hfft", "ihfft"):
    globals()[_name] = _no_complex(_name)
del _name


def fftfreq(n, d=1.0, *, device=None):
    """Sample frequencies [0, 1, ..., ceil(n/2)-1, -floor(n/2), ..., -1] / (d n)."""
    from .creation import arange
    from .manipulation import concatenate
    val = 1.0 / (n * d)
    N = (n - 1) // 2 + 1
    idx = concatenate([arange(0, N, dtype=np.int64), arange(-(n // 2), 0, dtype=np.int64)])
    return idx * val


def rfftfreq(n, d=1.0, *, device=None):
    from .creation import arange
    return arange(0, n // 2 + 1, dtype=np.int64) * (1.0 / (n * d))


def _shift(x, axes, sign):
    from .creation import asarray
    from .manipulation import roll
    a = asarray(x)
    if axes is None:
        axes = tuple(range(a.ndim))
        shift = [sign * (dim // 2) for dim in a.shape]
    elif isinstance(axes, (int, np.integer)):
        shift = sign * (a.shape[axes] // 2)
    else:
        shift = [sign * (a.shape[ax] // 2) for ax in axes]
    return roll(a, shift, axes)


def fftshift(x, axes=None):
    """Zero frequency moved to the centre (a roll by n // 2 per axis)."""
    return _shift(x, axes, 1)


def ifftshift(x, axes=None):
    return _shift(x, axes, -1)
