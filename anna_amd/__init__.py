"""MI355X-native implementation of Anna's quantized decode path.

Group-wise int4 weight-only linear, TurboQuant KV-cache packing and GQA decode
attention over the packed cache, as hand-written HIP kernels for gfx950 behind the
reference's Python module API and ``anna::`` op schemas.
"""

__all__ = ["fused_ops", "quantization"]
