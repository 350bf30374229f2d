"""Host wrappers of the gfx950 HIP kernels (C ABI: include/oscar_amd.h)."""
