"""pie_amd: MI355X (gfx950) kernels for the per-layer hot path of Pie's Python backend.

``pie_amd.ops`` is the drop-in op namespace (flashinfer names + the inline torch expressions
of the model files); ``pie_amd.integration`` installs it under the names the model files
import. Kernels live in ``libpie_hip.so`` (C ABI in include/pie_hip.h), built by
``python -m pie_amd.build``.
"""
from . import ops  # noqa: F401

__all__ = ["ops"]
__version__ = "0.1.0"
