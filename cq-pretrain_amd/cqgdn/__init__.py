"""cqgdn - MI355X (gfx950) gated delta-rule backend, selected as ``gdn_backend: hip``.

``cqgdn.gated_delta_net`` mirrors the reference's ``ops/gated_delta_net.py``; the
kernels live in ``libcqgdn.so`` (C ABI: include/cqgdn.h).
"""

from . import gated_delta_net
from .gated_delta_net import delta, initialize, prefill, provenance, recurrent

__all__ = ["gated_delta_net", "delta", "initialize", "prefill", "provenance", "recurrent"]
