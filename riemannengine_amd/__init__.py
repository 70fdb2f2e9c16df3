"""MI355X-native sparse-convolution hot path of RiemannEngine.

Coordinate hashing, kernel-map generation and gather-GEMM-scatter sparse
convolution (forward, dX, dW) as hand-written gfx950 HIP kernels behind the C
ABI in include/riemann_hip.h (libriemann_hip.so). ``abi`` binds that ABI with
ctypes over torch device memory; ``stencil`` enumerates convolution offsets;
``scenes`` generates the seeded benchmark point clouds.
"""
__version__ = "0.1.0"
