"""kernelforge: KernelForge's tunable kernel set, rebuilt for MI355X (gfx950).

Importing the package loads no GPU code: the HIP library
(``libkernelforge_hip.so``) is loaded on the first kernel call, and the kernel
modules are resolved lazily through :mod:`kernelforge.kernels`.
"""

__version__ = "0.1.0"
