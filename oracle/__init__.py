"""CPU oracle for the tree-attention path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference computes on the path the
HIP engine replaces: DFS tree metadata, partitioning and gateway biases, and
dense-mask attention forward/backward. Every function cites the reference
file:line it follows (``dfs_tree_forward.py``, ``tree_grad_hybrid.py``,
``tree_grad_ckpt.py``, ``tree_grad_ckpt_opath.py`` of Jinghui-Wang/tree-training,
and the transformers source the reference calls for attention arithmetic).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or the timed CPU
baseline. The product package ``tree_training_amd`` never imports it.

Pinning (what fixes each function independently of its own formula):
  * tree_meta.build_dfs_tree_info_literal / meta_closed_form — hand-traced
    fixtures (47-token two-root tree; 5-node chain tree), brute-force ancestor
    walk on random forests, literal-vs-closed-form agreement, nnz = sum(pos+1).
  * partition.partition_tree_literal / gateway_bias — hand-traced partition
    sizes and gateway biases for max_tokens in {1000, 20, 10, 6}, plus the
    disjoint-cover / budget / parent-before-child invariants.
  * attention.attn_fwd / attn_bwd — torch.nn.functional.scaled_dot_product_attention
    and torch autograd (library routines), finite differences, and per-path
    equivalence (tree rows == plain causal attention over each root-to-leaf path).
  * gdn — transformers' gated-delta-rule routines and module (library), conv1d
    on every path, finite differences; see oracle/gdn.py.
  * prologue.qk_prologue — transformers' Qwen3RMSNorm + apply_rotary_pos_emb and
    their autograd gradients (library), in float64.
"""
