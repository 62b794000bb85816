"""HIP-backed eager operators with the reference's signatures (flashquest.eager)."""
from .criticality import (  # noqa: F401
    page_scores, page_scores_int4_fast, page_scores_int8, page_scores_int8_fast, page_scores_int8_summary,
)
from .decode import (  # noqa: F401
    QuestDecoder, bf16_dense_attn_with_lse, merge_two_attentions, quest_decode_int4, quest_decode_int8,
    quest_decode_turbo,
    sparse_decode_layer,
)
from .page_summary import compute_page_summary  # noqa: F401
from .prefill import prefill_attention_layer  # noqa: F401
from .selection import build_compact_selection, select_pages, select_pages_vectorized  # noqa: F401
