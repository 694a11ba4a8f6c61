"""kernelo_amd: KernelForge's tunable kernel set, rebuilt for MI355X (gfx950).

Importing the package loads no GPU code: the HIP library
(``libkernelo_amd.so``) is loaded on the first kernel call, and the kernel
modules are resolved lazily through :mod:`kernelo_amd.kernels`.
"""

__version__ = "0.1.0"
