"""MI355X-native SE12 fused decode + GEMV (gfx950 HIP kernels behind a C ABI).

Modules: `format` (SE12 types, mirror of the reference domain), `launch`
(launch configurations and tuner rules), `hip` (the GPU adapters), `_native`
(ctypes binding of libse12_gfx950.so).
"""

__version__ = "0.1.0"
