"""MI355X (gfx950) implementation of BoaConstrictor's batched compress/decompress hot path.

Layout of the package directory ``boa-constrictor_amd/``:
  boa.py, codec.py, model.py, gpu_range_coder.py -- drop-in modules with the reference's names and APIs
  boa_amd/                                       -- ctypes binding of libboa_hip.so, weights, build recipe
  csrc/                                          -- HIP kernels (gfx950) and the C ABI (include/boa_hip.h)
"""
