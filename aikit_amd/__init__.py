"""aikit_amd -- MI355X (gfx950) W8A8 linear engine for aikit's encoder seam.

``libenchip.so`` (built from ``csrc/`` by ``build.py``) is the product: a C-ABI
library declared in ``include/enchip.h``. ``enchip`` is its ctypes binding.
"""
__all__ = ["enchip", "build"]
