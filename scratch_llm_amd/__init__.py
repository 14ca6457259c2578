"""scratch_llm's quantized-linear path, MI355X-native (gfx950 HIP kernels behind a C ABI).

``scratch_llm_amd.quant`` mirrors ``scratch_llm.quant`` (int4_group, int8, awq, nvfp4_mxfp4) on
ROCm device tensors; ``libsqx_hip.so`` (include/sqx.h) holds the kernels.
"""

__version__ = "0.1.0"
