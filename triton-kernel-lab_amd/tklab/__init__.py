"""tklab for AMD Instinct MI355X (gfx950).

The package keeps the module layout and public entry points of
triton-kernel-lab's ``tklab`` (reference ``src/tklab/__init__.py:1-12``) while
every device kernel is a hand-written HIP kernel in ``libtklab_hip.so``.
"""

from tklab.registry import REGISTRY, KernelSpec, register

__version__ = "0.1.0+mi355x"

__all__ = ["REGISTRY", "KernelSpec", "__version__", "register"]
