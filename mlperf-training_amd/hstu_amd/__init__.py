"""MI355X-native (gfx950) HSTU hot path: jagged causal SiLU attention (bf16 and
FP8 e4m3), the FP8 projections around it and the output block's
LayerNorm * U * dropout, behind the reference's op signatures.  Kernels live in ``libhstu_mi355x.so`` (C ABI, include/hstu_mi355x.h)."""

from ._lib import HstuKernelError, HstuUnavailableError, load_library  # noqa: F401
from .hstu_attention import (  # noqa: F401
    HammerKernel,
    hstu_mha,
    triton_hstu_attention_bwd,
    triton_hstu_attention_fwd,
    triton_hstu_mha,
    try_hstu_attention_bwd,
    try_hstu_attention_fwd,
    unsupported_shape_reason,
)
from .hstu_linear import (  # noqa: F401
    HSTUComputeOutputFunction,
    LayerNormMulDropoutFunction,
    create_dropout_mask,
    hstu_compute_output,
    triton_hstu_compute_output,
    triton_layer_norm_mul_dropout_bwd,
    triton_layer_norm_mul_dropout_fwd,
    triton_norm_mul_dropout,
    triton_weighted_layer_norm_bwd,
    triton_weighted_layer_norm_fwd,
)
from .hstu_preprocess import (  # noqa: F401
    hstu_compute_uqvk,
    hstu_layer,
    hstu_preprocess_and_attention,
    triton_hstu_preprocess_and_attention,
)
from .hstu_delta import delta_hstu_mha, triton_cached_hstu_mha, triton_hstu_attention_delta_bwd  # noqa: F401
from .hstu_do_fp8 import dequantize_do_e4m3_blk, quantize_do_e4m3_blk  # noqa: F401
from . import reference_ops  # noqa: F401,E402  (registers generative_recommenders::triton_hstu_attention_*)
