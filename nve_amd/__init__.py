"""nve_amd -- MI355X (gfx950) quantized decode GEMV path of genovationtech/nve.

The compute lives in libnve_hip.so (HIP kernels behind the C ABI declared in
include/nve_kernels.h).  This package holds the host-side mirror of the reference's
operator API for that path:

  nve_amd.hip_kernels  -- the wrappers of src/cuda_kernels.rs (quantize_f16_q8,
                          matvec_w4a8, fused_matvec_w4a16, fused_qkv_matvec_w4a16,
                          the _into variants) over torch device tensors
  nve_amd.gpu_layer    -- GpuW4 upload (ws_to_gpu) and the per-layer W4A8/W4A16
                          precision dispatch (src/gpu_layer.rs)

There is no CPU fallback: every entry point raises if libnve_hip.so is missing.
"""
from ._lib import NveError, lib, LIB_PATH  # noqa: F401

__all__ = ["NveError", "lib", "LIB_PATH"]
