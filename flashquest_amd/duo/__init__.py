"""DuoAttention head patterns (src/flashquest/duo/): retrieval heads select
pages by score, streaming heads keep only the sink and window pages."""
from .fused_dispatch import quest_duo_fused_sdpa
from .pattern import load_duo_pattern

__all__ = ["load_duo_pattern", "quest_duo_fused_sdpa"]
