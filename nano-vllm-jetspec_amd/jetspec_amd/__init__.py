"""MI355X-native tree-verification hot path of nano-vllm-jetspec.

Drop-in operators (same names, arguments and errors as the reference):
  packed_tree_attention   speculative/jetspec/paged_backend.py:240-306
  store_kvcache           layers/attention.py:38-45
  copy_accepted_kv        speculative/jetspec/state.py:64-86
  PackedTreeMetadata      speculative/jetspec/packed_metadata.py:16-237
  accept_batch            speculative/jetspec/serving_ops.py:55-90
  rope_scatter(_prevalidated)  speculative/jetspec/tree_fusion.py:167-199
  offset_causal_mask      speculative/jetspec/prefill.py:14-26 (a chunk is a chain tree)
Each device operator is a hand-written gfx950 HIP kernel in libtreeverify.so.
"""
from .packed_metadata import PackedTreeMetadata
from .paged_backend import packed_tree_attention, paged_tree_attention
from .tree_attention import packed_tree_attention_reference, packed_tree_attention_register_tuned
from .tree_dot import packed_tree_attention_dot
from .tree_gqa import packed_tree_attention_gqa
from .tree_prefix import (
    packed_tree_attention_prefix,
    packed_tree_attention_prefix_prevalidated,
    packed_tree_attention_prefix_single_loop,
    packed_tree_attention_prefix_split_exact,
)
from .attention import store_kvcache
from .tree_fusion import rope_scatter, rope_scatter_prevalidated
from .prefill import chain_tree_masks, offset_causal_mask
from .state import commit_slots, copy_accepted_kv, _slots_for_blocks
from .serving_ops import (accept_batch, accept_batch_device, accept_walk, build_child_maps, greedy_argmax,
                          truncate_accepted)
from ._device import read_and_clear_status
from ._lib import library

__all__ = [
    "PackedTreeMetadata",
    "packed_tree_attention",
    "packed_tree_attention_dot",
    "packed_tree_attention_gqa",
    "packed_tree_attention_prefix",
    "packed_tree_attention_prefix_single_loop",
    "packed_tree_attention_prefix_prevalidated",
    "packed_tree_attention_prefix_split_exact",
    "packed_tree_attention_reference",
    "packed_tree_attention_register_tuned",
    "paged_tree_attention",
    "store_kvcache",
    "rope_scatter",
    "rope_scatter_prevalidated",
    "offset_causal_mask",
    "chain_tree_masks",
    "copy_accepted_kv",
    "commit_slots",
    "accept_batch",
    "accept_batch_device",
    "greedy_argmax",
    "accept_walk",
    "truncate_accepted",
    "build_child_maps",
    "read_and_clear_status",
    "library",
]
