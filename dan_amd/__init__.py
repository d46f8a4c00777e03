"""dan_amd: gfx950 (MI355X) tree-masked prefill attention for dan-style packed reads.

``dan_amd.attention`` is the drop-in for dan/attention.py; its ``attend`` runs
one fused HIP kernel (dan_amd/csrc/tree_attn.hip) through the C ABI declared in
include/dan_tree_attn.h.
"""
from .attention import Batch, Segment, attend, branch_rows_mask, repeat_heads, segment, to_device, tree_mask

__all__ = ["Batch", "Segment", "attend", "branch_rows_mask", "repeat_heads", "segment", "to_device", "tree_mask"]
