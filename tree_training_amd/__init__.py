"""MI355X tree-attention engine for Tree Training (drop-in for Jinghui-Wang/tree-training).

Public API (same names and signatures as the reference modules):
  TreeNode, DFSTreeInfo, build_dfs_tree_info          (dfs_tree_forward.py Parts 1-2)
  DFSTreeResult, dfs_tree_forward                     (dfs_tree_forward.py Parts 7-8)
  tree_grad_ckpt_sequential                           (tree_grad_ckpt.py)
  SubtreePartition, partition_tree, SubtreeGateway,
  tree_grad_hybrid, make_tree_loss_fn                 (tree_grad_hybrid.py)
  GatewayCache                                        (tree_grad_ckpt_opath.py)
The attention runs in hand-written HIP kernels for gfx950 (tree_training_amd/csrc),
reached through the C ABI of include/tree_attn.h.
"""
from .tree import DFSTreeInfo, TreeNode, build_dfs_tree_info
from .dfs_tree_forward import DFSTreeResult, dfs_tree_forward
from .ckpt import tree_grad_ckpt_sequential
from .hybrid import (SubtreeGateway, SubtreePartition, make_tree_loss_fn, partition_tree,
                     tree_grad_hybrid)
from .gateway import GatewayCache

__all__ = [
    "TreeNode", "DFSTreeInfo", "build_dfs_tree_info", "DFSTreeResult", "dfs_tree_forward",
    "tree_grad_ckpt_sequential", "SubtreePartition", "partition_tree", "SubtreeGateway",
    "tree_grad_hybrid", "make_tree_loss_fn", "GatewayCache",
]
