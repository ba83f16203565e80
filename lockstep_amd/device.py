"""Device guard: the HIP kernels here are built for gfx950 (MI355X) only.

Same contract as the reference's h100.py:8-15 require_h100(): return GPU 0's
properties, or exit with a message naming what was found.
"""

import sys

import torch


def require_gfx950():
    """Return GPU 0's properties, or exit unless it is a gfx950 (MI355X class)."""
    if not torch.cuda.is_available():
        sys.exit("needs an MI355X (gfx950): no HIP device")
    p = torch.cuda.get_device_properties(0)
    arch = getattr(p, "gcnArchName", "")
    if not arch.startswith("gfx950"):
        sys.exit(f"needs an MI355X (gfx950): found {p.name} ({arch or 'unknown arch'})")
    return p
