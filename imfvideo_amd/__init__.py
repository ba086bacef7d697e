"""MI355X (gfx950) SLA2 INT8 cube-attention hot path.

Modules mirror the reference's models/ files for this path:
  imfvideo_amd.sla2_cube_qat          <- models/sla2_cube_qat.py
  imfvideo_amd.mla_video_sparse_jvp   <- models/mla_video_sparse_jvp.py (router, tiling)
  imfvideo_amd.kernel_sparse_qat      <- models/sla2_vendor/kernel_sparse_qat.py (quantize_qkv)
The compute runs in libsla2hip.so (include/sla2h.h); ``imfvideo_amd.ops``
holds the torch-facing wrappers of its entry points.
"""

__version__ = "0.1.0"
