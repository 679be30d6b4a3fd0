"""Speculative decoding API (mirrors ``flashgrpo.decoding``)."""
from .acceptance import exact_accept_path, exact_accept_paths_batch, logits_to_probs, sample_from_logits
from .flash_medusa_decoder import FlashMedusaConfig, FlashMedusaDecoder
from .kv_extraction import KvExtractionResult, extract_accepted_path_kv
from .medusa_tree import (CandidateTree, TreePlan, TreeTopology, build_batch_trees, build_dense_tree,
                          dense_node_count, fit_topk_to_budget, plan_tree)
from .tree_attention import build_tree_attention_inputs, tree_ancestor_bits

__all__ = ["CandidateTree", "TreePlan", "TreeTopology", "FlashMedusaConfig", "FlashMedusaDecoder",
           "KvExtractionResult", "build_batch_trees", "build_dense_tree", "build_tree_attention_inputs",
           "dense_node_count", "exact_accept_path", "exact_accept_paths_batch", "extract_accepted_path_kv",
           "fit_topk_to_budget", "logits_to_probs", "plan_tree", "sample_from_logits", "tree_ancestor_bits"]
