"""puffysics_amd - MI355X-native batched rigid-body stepping for Puffysics.

The product is libb3engine.so (gfx950 HIP kernels behind the C ABI of
include/b3_engine.h); this package is its Python host side:
  b3types  ctypes / numpy mirrors of B3World and friends
  scenes   the five benchmark world families and their host builders
  engine   B3Engine and the b3_batch_*_gpu functions
"""
from .b3types import signature, world_dtype, world_size  # noqa: F401
