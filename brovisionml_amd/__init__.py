"""brovisionml_amd -- MI355X (gfx950) DSINE surface-normal ops.

The native product is brovisionml_amd/lib/libbvml_dsine.so (HIP kernels,
the C ABI of include/bvml_dsine.h and the C++ drop-in of
include/brovisionml/dsine_ops.h).  This package is the Python host side:
  brovisionml_amd.dsine      ray_relu / angmf_propagate on device tensors
  brovisionml_amd._lib       raw ctypes binding of the C ABI
  brovisionml_amd.workloads  synthetic inputs and camera closed forms
  brovisionml_amd.build      hipcc build recipe
"""
from . import _lib, dsine, workloads  # noqa: F401

__version__ = "0.1.0"
