"""Versioned identities and thresholds of the MI355X MoE path.

Thresholds keep the reference's values (glm53_flash_mlx/abi.py:5-6): the
grouped prefill engages at 256 routes and the measured crossover is 16.
The ABI strings name this build's kernels and bank layout.
"""

GROUPED_MEASURED_CROSSOVER_ROUTES = 16
GROUPED_MIN_ROUTES = 256

KERNEL_ABI_VERSION = "glm53-mi355x-fp8-v1-e4m3f16-dot2-gemv"
GROUPED_KERNEL_ABI = "glm53-mi355x-grouped-fp8-v1-mfma16x16x128-hilo"
PACKED_EXPERT_BANK_ABI = "glm53-packed-expert-bank-v2-gate-up-output-major-row-contiguous"
PACKED_DECODE_KERNEL_ABI = "glm53-mi355x-packed-decode-v1-fused-gate-up-swiglu-down-reduce-shared"
NATIVE_C_ABI_VERSION = 1
