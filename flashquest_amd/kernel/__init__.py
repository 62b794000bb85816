"""HIP-backed kernels with the reference's operator signatures (flashquest.kernel)."""
from .kv_quant import (  # noqa: F401
    dequantize_k, dequantize_k_int4, dequantize_v, dequantize_v_int4, quantize_k, quantize_k_int4,
    quantize_k_turbo, quantize_v, quantize_v_int4, quantize_v_turbo,
)
from .prefill import flash_attn_prefill_int4, flash_attn_prefill_int8, flash_attn_prefill_turbo  # noqa: F401
from .sparse_fwd import flash_attn_sparse_fwd  # noqa: F401
from .sparse_int4_fwd import flash_attn_sparse_int4_fwd  # noqa: F401
from .sparse_int4_fwd_compact import flash_attn_sparse_int4_fwd_compact  # noqa: F401
from .sparse_turbo_fwd import flash_attn_sparse_turbo_fwd  # noqa: F401
from .wht import wht_along_head_dim  # noqa: F401
