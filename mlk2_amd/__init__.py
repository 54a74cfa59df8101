"""MI355X-native (gfx950) execution backend for MLK+ KernelModules.

The product is ``lib/libmlk_hip.so``: hand-written HIP kernels for the
recognized KernelModule classes behind a C ABI (``include/mlk_hip.h``). The
Python modules here mirror the reference's host interface (Kernel IR data
model, module builders, the driver's LoadedKernel) over that ABI.
"""
