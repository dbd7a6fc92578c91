"""ironmill_amd -- MI355X (gfx950) backend for ironmill's quantized-decode path.

The work happens in ``lib/libironmill_hip.so`` (hand-written HIP kernels behind
the C ABI of ``include/ironmill_hip.h``); this package is its Python face:

* ``runtime``: Device / Buffer / Stream / Event (the ironmill-metal-sys tier),
* ``ops``: the op encoders (INT4 projections, fused gate+up, fused residual
  norm projection, TurboQuant cache write and decode attention),
* ``quant``: the host-side INT4 quantizer that produces the weight layout,
* ``bundle``: the `.ironml-gpu` bundle reader (and writer) and a decoder
  built from a bundle.
"""
from ._lib import IronmillError, LIB_PATH  # noqa: F401  (raises if the library is missing)
from . import bundle, ops, quant, runtime  # noqa: F401
from .runtime import Buffer, Device, Event, Stream  # noqa: F401

__all__ = ["IronmillError", "LIB_PATH", "bundle", "ops", "quant", "runtime", "Device", "Buffer", "Stream", "Event"]
