"""HIP kernels for gfx950 behind a C ABI (include/rk_path.h), built into librk_path.so and bound with ctypes."""
