"""nurostream_amd: the MoE expert hot path of neurostream, native to MI355X (gfx950).

Compute runs in hand-written HIP kernels (libnsx.so, C ABI in
include/nurostream_amd.h); this package mirrors the reference's Python seams
(compute.quant.dequantize, compute.kernels.fused_gemv, compute.blockffn.*,
moe.router, model.gpt_oss, residency.cache.TieredCache, io.*, api.NeuroStream).
"""
__version__ = "0.1.0"
