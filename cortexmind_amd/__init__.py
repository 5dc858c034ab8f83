"""CortexMind MI355X (gfx950) backend: hand-written HIP kernels behind the C
ABI in include/cxm_hip.h, with a Python mirror of the reference engine's
operator structs (cortexmind_amd.engine) for tests and benchmarks.

Importing the package does not load the library; ``cortexmind_amd._lib.lib()``
does, and raises if it has not been built.
"""
__version__ = "0.1.0"
