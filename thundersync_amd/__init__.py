"""MI355X-native (gfx950 HIP) kernels for thundersync's hot path.

Operators keep the reference's Python API (seilk/thundersync,
``thundersync.accel`` and the attention dispatch of
``thundersync.engine.streaming``) so its streaming engine can call them as a
drop-in behind the ``THUNDERSYNC_HIP`` switch.  Submodules import lazily.
"""

from __future__ import annotations

__version__ = "0.1.0"
