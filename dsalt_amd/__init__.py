"""MI355X-native DSALT sparse attention (gfx950 HIP kernels behind a C ABI).

Layout:
  dsalt_amd.ops        torch-tensor wrappers of the C ABI (include/dsalt_amd.h)
  dsalt_amd.kernels    the reference library's kernel-level API (dsalt.kernels names)
  dsalt_amd.modules    DSALTAttention (inference path of the reference module)
  dsalt_amd.workloads  seeded synthetic inputs of the benchmarked workloads
"""
__version__ = "0.1.0"
