"""MI355X (gfx950) forward renderer for neural shell texture splatting.

The compute path is libnest_splat.so (HIP kernels behind the C ABI of
include/nest_splat.h); this package holds the host side: the ctypes binding,
scene and camera helpers, the MLP and RVQ modules and the render() driver.
"""
