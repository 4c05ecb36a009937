"""CPU oracle of the tree-verify hot path - test infrastructure only (see oracle.py)."""
from .oracle import *  # noqa: F401,F403
from .oracle import (accept_walk, argmax_flip_witness, child_maps, copy_accepted_kv, fp64_attention,
                     mask_from_parents, metadata_arrays, metadata_tree_attention_f64, parent_chain,
                     rope_hf_order, rope_scatter_hf, store_kvcache, tree_attention_f64)
