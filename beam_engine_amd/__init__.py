"""beam_engine_amd: MI355X-native beam-search decode hot path.

Drop-in for the decode path of brian030128/beam_engine: paged KV cache and
allocator (``PageTable``), beam trie (``BeamState``), flat / cascade decode
and paged prefill attention wrappers, and GPU beam selection (vanilla and
diverse), all backed by hand-written gfx950
HIP kernels in ``libbeam_engine_amd.so`` (C ABI: include/beam_engine_amd.h).
There is no CPU fallback: every compute call raises if the library is missing.
"""

from .attention import (BatchDecodeWithPagedKVCacheWrapper, BatchPrefillWithPagedKVCacheWrapper,
                        MultiLevelCascadeAttentionWrapper, merge_state)
from .attention_mode import AttentionMode
from .beam_state import (BeamCandidate, BeamGenerateInput, BeamGenerateResult, BeamState, BeamToken,
                         BeamTokenCandidate, TrieNode)
from .beam_strategy import BeamStrategy, DiverseBeamSearchStrategy, VanillaBeamSearchStrategy
from .kv_tree_node import KVTreeNode
from .page_table import PageTable
from .selection import beam_topk, decode_k

__all__ = [
    "AttentionMode", "BatchDecodeWithPagedKVCacheWrapper", "BatchPrefillWithPagedKVCacheWrapper", "BeamCandidate",
    "BeamGenerateInput",
    "BeamGenerateResult", "BeamState", "BeamStrategy", "BeamToken", "BeamTokenCandidate", "KVTreeNode",
    "MultiLevelCascadeAttentionWrapper", "PageTable", "TrieNode", "VanillaBeamSearchStrategy",
    "DiverseBeamSearchStrategy", "beam_topk",
    "decode_k", "merge_state",
]

__version__ = "0.1.0"
