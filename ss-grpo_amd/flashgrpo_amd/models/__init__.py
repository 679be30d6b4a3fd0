"""Model adapters (mirrors ``flashgrpo.models``): Medusa heads and the native target model."""
from .medusa_heads import ChainDraftCell, MedusaHeads, MedusaPredictionHead
from .target import KVCache, TargetConfig, TargetModel, forward_tree

__all__ = ["ChainDraftCell", "MedusaHeads", "MedusaPredictionHead", "KVCache", "TargetConfig", "TargetModel",
           "forward_tree"]
