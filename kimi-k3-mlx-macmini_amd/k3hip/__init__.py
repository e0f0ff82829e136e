"""k3hip: MI355X (gfx950) native MXFP4 expert / latent-MLA decode hot path.

Host-side mirror of the reference interfaces, backed by hand-written HIP kernels in
``libk3hip.so`` (C-ABI: ``include/k3hip.h``):

* ``k3hip.mxfp4``          decode_mxfp4 / decode_scale / assert_scales_representable /
                           mxfp4_matvec        (air_llm/models/kimi_k3/mxfp4.py)
* ``k3hip.mxfp4_matvec``   mxfp4_matvec_fused / expert_projection
                           (air_llm/kernels/metal/mxfp4_matvec.py)
"""
from __future__ import annotations

from ._lib import K3LibraryError, LIB_PATH, lib  # noqa: F401

__all__ = ["K3LibraryError", "LIB_PATH", "lib"]
