"""ctypes binding of the C ABI in include/tree_attn.h.

The shared library is built in-tree (``python -m tree_training_amd.build``)
into ``tree_training_amd/lib/libtree_attn.so``. Loading fails loudly when it is
missing: there is no CPU fallback for any entry point.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# TREE_ATTN_LIB selects an alternate build of the same library (A/B timing).
LIB_PATH = os.environ.get("TREE_ATTN_LIB") or os.path.join(_HERE, "lib", "libtree_attn.so")

TT_OK = 0
TT_E_ARG = -1
TT_E_UNSUPPORTED = -2
TT_E_HIP = -3
TT_E_WORKSPACE = -4
TT_DTYPE_F32 = 0
TT_DTYPE_BF16 = 1
TT_BWD_DELTA = 1
TT_BWD_DQ = 2
TT_BWD_DKDV = 4
TT_BWD_DETERMINISTIC = 8
TT_STATUS_BAD_LEN = 1
TT_STATUS_BAD_PARENT = 2
TT_STATUS_BAD_TOTAL = 4
TT_STATUS_BAD_BIAS = 8

ABI_VERSION = 9

# Every symbol include/tree_attn.h declares, for the export check.
EXPORTS = (
    "tt_abi_version", "tt_strerror", "tt_meta_workspace_bytes", "tt_meta_build", "tt_keys_build",
    "tt_meta_dense_mask", "tt_plan_bytes", "tt_plan_build", "tt_attn_fwd_workspace_bytes", "tt_attn_fwd",
    "tt_attn_bwd_workspace_bytes", "tt_attn_det_slots", "tt_attn_split_tiles", "tt_attn_bwd", "tt_gdn_workspace_bytes", "tt_gdn_tree_fwd",
    "tt_gdn_bwd_workspace_bytes", "tt_gdn_tree_bwd", "tt_gdn_saved_bytes", "tt_gdn_tree_fwd_save",
    "tt_gdn_bwd_saved_workspace_bytes", "tt_gdn_tree_bwd_saved", "tt_tree_conv_fwd", "tt_tree_conv_bwd_workspace_bytes",
    "tt_tree_conv_bwd", "tt_qk_prologue_fwd", "tt_qk_prologue_bwd_workspace_bytes", "tt_qk_prologue_bwd", "tt_ce_rows",
    "tt_selftest_mfma32", "tt_noalloc_scratch_bytes", "tt_attn_bwd_noalloc", "tt_trees_build",
)

TT_TREE_JOBS_MAX = 16


class TTTensor(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_void_p), ("stride_tok", ctypes.c_int64), ("stride_head", ctypes.c_int64)]


class TTTreeJob(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "node_len", "node_parent", "past_bias", "node_start", "node_off", "node_hend", "pos", "node_of", "horizon",
        "key_lo", "key_hi", "status", "plan")] + [("plan_bytes", ctypes.c_size_t), ("ws", ctypes.c_void_p),
                                                   ("ws_bytes", ctypes.c_size_t)] + \
        [(n, ctypes.c_int32) for n in ("n_nodes", "n_tokens", "pos_offset", "n_past")]


class TTAttnProblem(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("n_q", ctypes.c_int32), ("n_past", ctypes.c_int32),
        ("n_heads_q", ctypes.c_int32), ("n_heads_kv", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("scale", ctypes.c_float), ("bwd_parts", ctypes.c_int32),
        ("q", TTTensor), ("k", TTTensor), ("v", TTTensor), ("k_past", TTTensor), ("v_past", TTTensor),
        ("key_lo", ctypes.c_void_p), ("key_hi", ctypes.c_void_p), ("plan", ctypes.c_void_p),
        ("plan_bytes", ctypes.c_size_t), ("det_slots", ctypes.c_int64), ("split_tiles", ctypes.c_int64),
    ]


class TTGdnProblem(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("n_tokens", ctypes.c_int32), ("n_nodes", ctypes.c_int32),
        ("n_heads_k", ctypes.c_int32), ("n_heads_v", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("l2norm", ctypes.c_int32), ("scale", ctypes.c_float),
        ("q", TTTensor), ("k", TTTensor), ("v", TTTensor),
        ("g", ctypes.c_void_p), ("g_stride_tok", ctypes.c_int64),
        ("beta", ctypes.c_void_p), ("beta_stride_tok", ctypes.c_int64),
        ("node_start", ctypes.c_void_p), ("node_len", ctypes.c_void_p), ("node_parent", ctypes.c_void_p),
        ("level_nodes", ctypes.c_void_p), ("level_offsets", ctypes.POINTER(ctypes.c_int32)),
        ("n_levels", ctypes.c_int32), ("n_chunks", ctypes.c_int32),
        ("node_chunk0", ctypes.c_void_p), ("chunk_node", ctypes.c_void_p),
        ("node_child_off", ctypes.c_void_p), ("node_child", ctypes.c_void_p),
        ("reference_truncated", ctypes.c_int32), ("initial_state", ctypes.c_void_p),
        ("d_states_last_only", ctypes.c_int32),
    ]


class TTConvProblem(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("n_tokens", ctypes.c_int32), ("n_channels", ctypes.c_int32),
        ("kernel_size", ctypes.c_int32), ("x", ctypes.c_void_p), ("x_stride_tok", ctypes.c_int64),
        ("weight", ctypes.c_void_p), ("bias", ctypes.c_void_p), ("tok_prev", ctypes.c_void_p),
        ("tok_next_off", ctypes.c_void_p), ("tok_next", ctypes.c_void_p),
    ]


class TTPrologueProblem(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("n_tokens", ctypes.c_int32), ("n_heads_q", ctypes.c_int32),
        ("n_heads_kv", ctypes.c_int32), ("head_dim", ctypes.c_int32), ("eps_q", ctypes.c_float),
        ("eps_k", ctypes.c_float), ("q", TTTensor), ("k", TTTensor), ("q_weight", ctypes.c_void_p),
        ("k_weight", ctypes.c_void_p), ("cos", ctypes.c_void_p), ("sin", ctypes.c_void_p),
        ("cs_stride_tok", ctypes.c_int64),
    ]


class TreeAttnError(RuntimeError):
    pass


_lib = None


def _declare(lib):
    P, I32, SZ, VP = ctypes.c_void_p, ctypes.c_int32, ctypes.c_size_t, ctypes.c_void_p
    sig = {
        "tt_abi_version": (ctypes.c_int, []),
        "tt_strerror": (ctypes.c_char_p, [ctypes.c_int]),
        "tt_meta_workspace_bytes": (SZ, [I32]),
        "tt_meta_build": (ctypes.c_int, [P, P, I32, I32, I32, P, P, P, P, P, P, P, P, SZ, VP]),
        "tt_keys_build": (ctypes.c_int, [P, I32, P, I32, P, P, P, VP]),
        "tt_meta_dense_mask": (ctypes.c_int, [P, P, I32, I32, P, VP]),
        "tt_plan_bytes": (SZ, [I32, I32]),
        "tt_plan_build": (ctypes.c_int, [P, P, I32, I32, P, SZ, VP]),
        "tt_trees_build": (ctypes.c_int, [ctypes.POINTER(TTTreeJob), I32, VP]),
        "tt_attn_fwd_workspace_bytes": (SZ, [ctypes.POINTER(TTAttnProblem)]),
        "tt_attn_fwd": (ctypes.c_int, [ctypes.POINTER(TTAttnProblem), P, P, P, SZ, VP]),
        "tt_attn_bwd_workspace_bytes": (SZ, [ctypes.POINTER(TTAttnProblem)]),
        "tt_attn_det_slots": (ctypes.c_int, [P, P, I32, P, I32, ctypes.POINTER(ctypes.c_int64)]),
        "tt_attn_split_tiles": (ctypes.c_int, [P, P, I32, P, I32, ctypes.POINTER(ctypes.c_int64)]),
        "tt_attn_bwd": (ctypes.c_int, [ctypes.POINTER(TTAttnProblem), P, P, TTTensor, P, P, P, P, P, P, SZ,
                                       VP]),
        "tt_gdn_workspace_bytes": (SZ, [ctypes.POINTER(TTGdnProblem)]),
        "tt_gdn_tree_fwd": (ctypes.c_int, [ctypes.POINTER(TTGdnProblem), P, P, P, SZ, VP]),
        "tt_gdn_bwd_workspace_bytes": (SZ, [ctypes.POINTER(TTGdnProblem)]),
        "tt_gdn_tree_bwd": (ctypes.c_int, [ctypes.POINTER(TTGdnProblem), TTTensor, TTTensor, TTTensor, TTTensor, P,
                                           P, P, P, P, SZ, VP]),
        "tt_gdn_saved_bytes": (SZ, [ctypes.POINTER(TTGdnProblem)]),
        "tt_gdn_tree_fwd_save": (ctypes.c_int, [ctypes.POINTER(TTGdnProblem), P, P, P, SZ, VP]),
        "tt_gdn_bwd_saved_workspace_bytes": (SZ, [ctypes.POINTER(TTGdnProblem)]),
        "tt_gdn_tree_bwd_saved": (ctypes.c_int, [ctypes.POINTER(TTGdnProblem), TTTensor, TTTensor, TTTensor, TTTensor,
                                                 P, P, P, P, P, SZ, P, SZ, VP]),
        "tt_tree_conv_fwd": (ctypes.c_int, [ctypes.POINTER(TTConvProblem), P, ctypes.c_int64, VP]),
        "tt_qk_prologue_fwd": (ctypes.c_int, [ctypes.POINTER(TTPrologueProblem), P, P, VP]),
        "tt_ce_rows": (ctypes.c_int, [I32, P, ctypes.c_int64, I32, I32, P, P, I32, P, P, ctypes.c_int64, VP]),
        "tt_qk_prologue_bwd_workspace_bytes": (SZ, [ctypes.POINTER(TTPrologueProblem)]),
        "tt_qk_prologue_bwd": (ctypes.c_int, [ctypes.POINTER(TTPrologueProblem), TTTensor, TTTensor, P, P, P, P, P,
                                              SZ, VP]),
        "tt_tree_conv_bwd_workspace_bytes": (SZ, [ctypes.POINTER(TTConvProblem)]),
        "tt_tree_conv_bwd": (ctypes.c_int, [ctypes.POINTER(TTConvProblem), P, ctypes.c_int64, P, P, P, P, SZ,
                                            VP]),
        "tt_selftest_mfma32": (ctypes.c_int, [P, P, P, VP]),
        "tt_noalloc_scratch_bytes": (SZ, []),
        "tt_attn_bwd_noalloc": (ctypes.c_int, [ctypes.POINTER(TTAttnProblem), P, P, TTTensor, P, P, P, P, P, VP]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


def lib():
    """Loads the HIP library (once). Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise TreeAttnError(
                f"{LIB_PATH} is missing: build it with `python -m tree_training_amd.build` "
                "(the tree-attention path has no CPU fallback)")
        l = ctypes.CDLL(LIB_PATH)
        _declare(l)
        v = l.tt_abi_version()
        if v != ABI_VERSION:
            raise TreeAttnError(f"libtree_attn ABI {v} != expected {ABI_VERSION}; rebuild the library")
        _lib = l
    return _lib


def check(rc: int, what: str):
    if rc != TT_OK:
        msg = lib().tt_strerror(rc).decode()
        raise TreeAttnError(f"{what} failed: {msg} (code {rc})")
