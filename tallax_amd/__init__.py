"""tallax_amd: MI355X-native (gfx950 HIP) sort / select / sample path of tallax.

Public modules mirror the reference: `tax` (tallax/tax.py), `tumpy`
(tallax/tumpy.py) and `sampling` (tallax/_src/sampling.py).
"""
from . import prefill, sampling, tax, tumpy  # noqa: F401

__all__ = ["tax", "tumpy", "sampling", "prefill"]
