"""mkernel_amd — MI355X (gfx950) compute core of mKernel's fused operators.

* ``mkernel_amd.capi``        ctypes binding of libmk's C-ABI (include/mk.h)
* ``mkernel_amd.ops``         torch-tensor front end (device memory/streams)
* ``mkernel_amd.load_module`` the reference's operator modules by name
  (``load("ag_gemm").ag_gemm_multinode(...)`` etc.)
* ``mkernel_amd.workloads``   seeded synthetic inputs of the BASELINE configs
"""
from .capi import MkError  # noqa: F401

__all__ = ["MkError"]
