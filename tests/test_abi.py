"""C-ABI checks that need no GPU: the library loads, exports every symbol the
header declares, and rejects bad arguments on the host before any launch."""
import ctypes
import os
import re

import pytest

from tree_training_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    src = open(os.path.join(ROOT, "include", "tree_attn.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(tt_[a-z0-9_]+)\s*\(", src)))


def test_exports_match_header():
    lib = _lib.lib()
    declared = header_symbols()
    assert declared == sorted(_lib.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name


def test_version_and_strerror():
    lib = _lib.lib()
    assert lib.tt_abi_version() == _lib.ABI_VERSION
    for code in (0, -1, -2, -3, -4, -99):
        assert lib.tt_strerror(code)


def _problem(**kw):
    p = _lib.TTAttnProblem(dtype=_lib.TT_DTYPE_BF16, n_q=100, n_past=0, n_heads_q=32, n_heads_kv=8,
                           head_dim=128, scale=128 ** -0.5, bwd_parts=0,
                           q=_lib.TTTensor(16, 32 * 128, 128), k=_lib.TTTensor(16, 8 * 128, 128),
                           v=_lib.TTTensor(16, 8 * 128, 128), k_past=_lib.TTTensor(None, 128, 128),
                           v_past=_lib.TTTensor(None, 128, 128), key_lo=16, key_hi=16, plan=16,
                           plan_bytes=_lib.lib().tt_plan_bytes(100, 100))
    for k, v in kw.items():
        setattr(p, k, v)
    return p


@pytest.mark.parametrize("field,value,code", [
    ("head_dim", 64, _lib.TT_E_UNSUPPORTED),
    ("dtype", 7, _lib.TT_E_UNSUPPORTED),
    ("n_heads_kv", 5, _lib.TT_E_UNSUPPORTED),
    ("n_q", 0, _lib.TT_E_ARG),
    ("scale", float("nan"), _lib.TT_E_ARG),
    ("scale", -1.0, _lib.TT_E_ARG),
    ("plan_bytes", 10, _lib.TT_E_WORKSPACE),
    ("key_lo", None, _lib.TT_E_ARG),
    ("n_past", 3, _lib.TT_E_ARG),            # past segment without pointers
])
def test_attn_fwd_validation(field, value, code):
    lib = _lib.lib()
    p = _problem(**{field: value})
    assert lib.tt_attn_fwd(ctypes.byref(p), ctypes.c_void_p(16), ctypes.c_void_p(16), None, 0, None) == code


def test_attn_stride_and_alignment_validation():
    lib = _lib.lib()
    p = _problem(q=_lib.TTTensor(16, 100, 128))         # stride not a multiple of 8
    assert lib.tt_attn_fwd(ctypes.byref(p), ctypes.c_void_p(16), ctypes.c_void_p(16), None, 0, None) == _lib.TT_E_ARG
    p = _problem(q=_lib.TTTensor(18, 32 * 128, 128))    # not 16-byte aligned
    assert lib.tt_attn_fwd(ctypes.byref(p), ctypes.c_void_p(16), ctypes.c_void_p(16), None, 0, None) == _lib.TT_E_ARG
    p = _problem()
    assert lib.tt_attn_fwd(ctypes.byref(p), None, ctypes.c_void_p(16), None, 0, None) == _lib.TT_E_ARG


def test_bwd_validation():
    lib = _lib.lib()
    p = _problem()
    ws = lib.tt_attn_bwd_workspace_bytes(ctypes.byref(p))
    assert ws >= 32 * 100 * 4
    d_o = _lib.TTTensor(16, 32 * 128, 128)
    V = ctypes.c_void_p(16)
    # one gateway accumulator without the other
    assert lib.tt_attn_bwd(ctypes.byref(p), V, V, d_o, V, V, V, V, None, V, ws, None) == _lib.TT_E_ARG
    # workspace too small
    assert lib.tt_attn_bwd(ctypes.byref(p), V, V, d_o, V, V, V, None, None, V, 8, None) == _lib.TT_E_WORKSPACE


def _qch(n_q):
    half = (1 << (n_q.bit_length() - 1)) // 2 if n_q >= 2 else 0
    return min(4096, max(256, half))


@pytest.mark.parametrize("n_q,n_past", [(100, 0), (600, 0), (16318, 0), (5300, 300), (50109, 0)])
def test_bwd_deterministic_workspace(n_q, n_past):
    """TT_BWD_DETERMINISTIC adds one dK and one dV slot of 128 keys x Hkv x
    128 fp32 for each possible work item beyond the first of a key tile:
    ceil(n_keys / 128) * floor((n_q - 1) / W) of them (W: the work item's
    query window); bf16 and fp32 problems share the layout up to the bf16
    dQ key-split partials of small problems."""
    lib = _lib.lib()
    base = _problem(n_q=n_q, n_past=n_past)
    det = _problem(n_q=n_q, n_past=n_past, bwd_parts=_lib.TT_BWD_DETERMINISTIC)
    n_kb = -(-(n_q + n_past) // 128)
    extra = 2 * n_kb * ((n_q - 1) // _qch(n_q)) * 128 * 8 * 128 * 4
    assert lib.tt_attn_bwd_workspace_bytes(ctypes.byref(det)) - \
        lib.tt_attn_bwd_workspace_bytes(ctypes.byref(base)) == extra
    assert (extra == 0) == (n_q <= 256 or n_q - 1 < _qch(n_q))
    sizes = [lib.tt_attn_bwd_workspace_bytes(ctypes.byref(p)) - _dq_part_bytes(n_q) for p in (base, det)]
    for p in (base, det):
        p.dtype = _lib.TT_DTYPE_F32
    assert [lib.tt_attn_bwd_workspace_bytes(ctypes.byref(p)) for p in (base, det)] == sizes


def _key_splits(n_q, hq=32):
    return 4 if -(-n_q // 128) * hq <= 256 else 1


def _r256(b):
    return (b + 255) // 256 * 256


def _dq_part_bytes(n_q, hq=32):
    s = _key_splits(n_q, hq)
    return _r256(s * n_q * hq * 128 * 4) if s > 1 else 0


@pytest.mark.parametrize("n_q,splits", [(1, 4), (100, 4), (473, 4), (1024, 4), (1025, 1), (1603, 1), (2048, 1),
                                        (16318, 1)])
def test_key_split_workspaces(n_q, splits):
    """Small bf16 problems (<= 256 pairs of 128-query block and q head) split
    the forward and dQ passes' keys in 4 ranges: the
    forward needs fp32 partial rows plus a row max and a row sum per split,
    the backward the dQ partial rows; fp32 problems and larger ones none."""
    lib = _lib.lib()
    assert _key_splits(n_q) == splits
    fwd = (_r256(splits * n_q * 32 * 512) + 2 * _r256(splits * 32 * n_q * 4)) if splits > 1 else 0
    p = _problem(n_q=n_q)
    assert lib.tt_attn_fwd_workspace_bytes(ctypes.byref(p)) == fwd
    f32 = _problem(n_q=n_q, dtype=_lib.TT_DTYPE_F32)
    assert lib.tt_attn_fwd_workspace_bytes(ctypes.byref(f32)) == 0
    assert lib.tt_attn_bwd_workspace_bytes(ctypes.byref(p)) - \
        lib.tt_attn_bwd_workspace_bytes(ctypes.byref(f32)) == _dq_part_bytes(n_q)


def test_attn_fwd_workspace_validation():
    """A split forward without its workspace: a null or misaligned ws is an
    argument error, a short one TT_E_WORKSPACE (checked before any launch)."""
    lib = _lib.lib()
    p = _problem(n_q=100)
    need = lib.tt_attn_fwd_workspace_bytes(ctypes.byref(p))
    assert need > 0
    V = ctypes.c_void_p(16)
    assert lib.tt_attn_fwd(ctypes.byref(p), V, V, None, need, None) == _lib.TT_E_ARG
    assert lib.tt_attn_fwd(ctypes.byref(p), V, V, ctypes.c_void_p(24), need, None) == _lib.TT_E_ARG
    assert lib.tt_attn_fwd(ctypes.byref(p), V, V, V, need - 4, None) == _lib.TT_E_WORKSPACE


def test_bwd_parts_validation():
    lib = _lib.lib()
    d_o = _lib.TTTensor(16, 32 * 128, 128)
    V = ctypes.c_void_p(16)
    p = _problem(bwd_parts=16)
    assert lib.tt_attn_bwd(ctypes.byref(p), V, V, d_o, V, V, V, None, None, V, 1 << 40, None) == _lib.TT_E_ARG


def test_bwd_noalloc_validation():
    """The no-allocation backward: a 96 MiB scratch, null problems rejected,
    and a problem whose workspace exceeds the scratch refused on the host
    (no HIP call: these run without a GPU)."""
    lib = _lib.lib()
    assert lib.tt_noalloc_scratch_bytes() == 96 << 20
    d_o = _lib.TTTensor(16, 32 * 128, 128)
    V = ctypes.c_void_p(16)
    assert lib.tt_attn_bwd_noalloc(None, V, V, d_o, V, V, V, None, None, None) == _lib.TT_E_ARG
    big = _problem(n_q=40000)
    assert lib.tt_attn_bwd_workspace_bytes(ctypes.byref(big)) > lib.tt_noalloc_scratch_bytes()
    assert lib.tt_attn_bwd_noalloc(ctypes.byref(big), V, V, d_o, V, V, V, None, None, None) == _lib.TT_E_WORKSPACE


@pytest.mark.parametrize("n_q,n_past", [(100, 0), (16318, 0), (5300, 300)])
def test_bwd_split_tiles_workspace(n_q, n_past):
    """The fp32 split sums take one dK and one dV block of 128 keys x Hkv x
    128 floats per split key tile the problem says it holds (split_tiles), or
    per key tile with split_tiles = 0; a negative count is an argument error."""
    lib = _lib.lib()
    n_kb = -(-(n_q + n_past) // 128)
    tile = 2 * 128 * 8 * 128 * 4
    full = _problem(n_q=n_q, n_past=n_past)
    some = _problem(n_q=n_q, n_past=n_past, split_tiles=3)
    assert lib.tt_attn_bwd_workspace_bytes(ctypes.byref(full)) - \
        lib.tt_attn_bwd_workspace_bytes(ctypes.byref(some)) == (n_kb - 3) * tile
    det = _problem(n_q=n_q, n_past=n_past, split_tiles=3, bwd_parts=_lib.TT_BWD_DETERMINISTIC, det_slots=2)
    assert lib.tt_attn_bwd_workspace_bytes(ctypes.byref(det)) - \
        lib.tt_attn_bwd_workspace_bytes(ctypes.byref(some)) == 2 * tile
    bad = _problem(n_q=n_q, n_past=n_past, split_tiles=-1, plan_bytes=lib.tt_plan_bytes(n_q, n_q + n_past),
                   k_past=_lib.TTTensor(16, 8 * 128, 128), v_past=_lib.TTTensor(16, 8 * 128, 128))
    assert lib.tt_attn_bwd_workspace_bytes(ctypes.byref(bad)) == 0
    d_o = _lib.TTTensor(16, 32 * 128, 128)
    V = ctypes.c_void_p(16)
    assert lib.tt_attn_bwd(ctypes.byref(bad), V, V, d_o, V, V, V, None, None, V, 1 << 40, None) == _lib.TT_E_ARG
    # the 16K agent tree's 14 split tiles fit the no-allocation scratch
    if n_q == 16318:
        tree = _problem(n_q=n_q, split_tiles=14)
        assert lib.tt_attn_bwd_workspace_bytes(ctypes.byref(tree)) < lib.tt_noalloc_scratch_bytes()


def _tree_job(**kw):
    V = 16
    j = _lib.TTTreeJob(**{n: V for n in ("node_len", "node_parent", "node_start", "node_off", "node_hend", "pos",
                                        "node_of", "horizon", "key_lo", "key_hi", "status", "plan", "ws")})
    j.past_bias = None
    j.n_nodes, j.n_tokens, j.pos_offset, j.n_past = 2, 10, 0, 0
    j.plan_bytes = _lib.lib().tt_plan_bytes(10, 10)
    j.ws_bytes = _lib.lib().tt_meta_workspace_bytes(2)
    for k, v in kw.items():
        setattr(j, k, v)
    return j


@pytest.mark.parametrize("kw,code", [
    (dict(n_nodes=0), _lib.TT_E_ARG),
    (dict(n_tokens=1), _lib.TT_E_ARG),                 # fewer tokens than nodes
    (dict(n_past=5), _lib.TT_E_ARG),                   # gateway without a bias
    (dict(pos=None), _lib.TT_E_ARG),
    (dict(plan_bytes=8), _lib.TT_E_WORKSPACE),
    (dict(ws_bytes=4), _lib.TT_E_WORKSPACE),
    (dict(n_tokens=70000, n_nodes=1), _lib.TT_E_UNSUPPORTED),   # beyond one workgroup per tree
])
def test_trees_build_validation(kw, code):
    """tt_trees_build checks every job on the host (no GPU call on these
    paths): sizes, pointers, buffer sizes and the batched limits."""
    lib = _lib.lib()
    jobs = (_lib.TTTreeJob * 2)(_tree_job(), _tree_job(**kw))
    assert lib.tt_trees_build(jobs, 2, None) == code


def test_trees_build_job_count():
    lib = _lib.lib()
    jobs = (_lib.TTTreeJob * 17)(*[_tree_job() for _ in range(17)])
    assert lib.tt_trees_build(jobs, 0, None) == _lib.TT_E_ARG
    assert lib.tt_trees_build(jobs, 17, None) == _lib.TT_E_ARG
    assert ctypes.sizeof(_lib.TTTreeJob) == 144


def test_binding_struct_sizes_match_the_header():
    """The ctypes structs have the sizes tt_api.hip asserts for the header's
    structs (a field missing on either side changes the size)."""
    sizes = dict(TTTensor=24, TTAttnProblem=200, TTGdnProblem=240, TTConvProblem=72, TTPrologueProblem=120,
                 TTTreeJob=144)
    for name, n in sizes.items():
        assert ctypes.sizeof(getattr(_lib, name)) == n, name


def test_meta_and_plan_validation():
    lib = _lib.lib()
    V = ctypes.c_void_p(16)
    assert lib.tt_meta_build(V, V, 0, 5, 0, V, V, V, V, V, V, V, V, 1 << 20, None) == _lib.TT_E_ARG
    assert lib.tt_meta_build(V, V, 3, 2, 0, V, V, V, V, V, V, V, V, 1 << 20, None) == _lib.TT_E_ARG
    assert lib.tt_meta_build(V, V, 3, 9, 0, V, V, V, V, V, V, V, V, 4, None) == _lib.TT_E_WORKSPACE
    assert lib.tt_meta_build(V, V, 3, 9, -1, V, V, V, V, V, V, V, V, 1 << 20, None) == _lib.TT_E_ARG
    assert lib.tt_keys_build(None, 4, V, 9, V, V, V, None) == _lib.TT_E_ARG
    assert lib.tt_plan_build(V, V, 5, 9, V, 1 << 20, None) == _lib.TT_E_ARG     # fewer keys than queries
    assert lib.tt_plan_build(V, V, 9, 9, V, 8, None) == _lib.TT_E_WORKSPACE
    assert lib.tt_plan_bytes(0, 5) == 0
    assert lib.tt_meta_workspace_bytes(0) == 0
    assert lib.tt_meta_dense_mask(V, V, 4, 70000, V, None) == _lib.TT_E_UNSUPPORTED


def _gdn_problem(offsets=(0, 1, 3), **kw):
    arr = (ctypes.c_int32 * len(offsets))(*offsets)
    p = _lib.TTGdnProblem(dtype=_lib.TT_DTYPE_BF16, n_tokens=100, n_nodes=3, n_heads_k=16, n_heads_v=32,
                          head_dim=128, l2norm=1, scale=128 ** -0.5,
                          q=_lib.TTTensor(16, 16 * 128, 128), k=_lib.TTTensor(16, 16 * 128, 128),
                          v=_lib.TTTensor(16, 32 * 128, 128), g=16, g_stride_tok=32, beta=16,
                          beta_stride_tok=32, node_start=16, node_len=16, node_parent=16, level_nodes=16,
                          level_offsets=arr, n_levels=len(offsets) - 1, n_chunks=5, node_chunk0=16,
                          chunk_node=16)
    p._keep = arr
    for k, v in kw.items():
        setattr(p, k, v)
    return p


@pytest.mark.parametrize("field,value,code", [
    ("head_dim", 64, _lib.TT_E_UNSUPPORTED),
    ("dtype", 7, _lib.TT_E_UNSUPPORTED),
    ("n_heads_v", 24, _lib.TT_E_UNSUPPORTED),     # not a multiple of n_heads_k
    ("n_tokens", 0, _lib.TT_E_ARG),
    ("n_nodes", 101, _lib.TT_E_ARG),             # more nodes than tokens
    ("scale", float("nan"), _lib.TT_E_ARG),
    ("g_stride_tok", 8, _lib.TT_E_ARG),           # rows of g overlap
    ("node_parent", None, _lib.TT_E_ARG),
    ("q", _lib.TTTensor(18, 16 * 128, 128), _lib.TT_E_ARG),   # misaligned
    ("reference_truncated", 2, _lib.TT_E_ARG),   # a flag: 0 or 1
    ("initial_state", 20, _lib.TT_E_ARG),        # misaligned
])
def test_gdn_validation(field, value, code):
    lib = _lib.lib()
    p = _gdn_problem(**{field: value})
    V = ctypes.c_void_p(16)
    assert lib.tt_gdn_tree_fwd(ctypes.byref(p), V, V, V, 1 << 30, None) == code


def test_gdn_reference_truncated_workspace():
    """The reference's per-node correction needs the node-level terms on top of
    the exact rule's workspaces: 32 decays and 32 x 256 R-rows per (chunk, v
    head) in the forward and saved buffers, and two more such rows plus the
    correction's dk and dG in the backward scratch."""
    lib = _lib.lib()
    ex, tr = _gdn_problem(), _gdn_problem(reference_truncated=1)
    ch = 5 * 32
    assert lib.tt_gdn_workspace_bytes(ctypes.byref(tr)) - lib.tt_gdn_workspace_bytes(ctypes.byref(ex)) == \
        ch * (32 + 32 * 256) * 4
    assert lib.tt_gdn_saved_bytes(ctypes.byref(tr)) - lib.tt_gdn_saved_bytes(ctypes.byref(ex)) == \
        ch * (32 + 32 * 256) * 4
    extra_scratch = ch * (2 * 32 * 256 + 32 * 128 + 32) * 4
    assert lib.tt_gdn_bwd_saved_workspace_bytes(ctypes.byref(tr)) - \
        lib.tt_gdn_bwd_saved_workspace_bytes(ctypes.byref(ex)) == extra_scratch
    assert lib.tt_gdn_bwd_workspace_bytes(ctypes.byref(tr)) - lib.tt_gdn_bwd_workspace_bytes(ctypes.byref(ex)) == \
        extra_scratch + ch * (32 + 32 * 256) * 4


def test_gdn_level_offsets_validation():
    lib = _lib.lib()
    V = ctypes.c_void_p(16)
    for offs in ((0, 2), (1, 3), (0, 2, 1, 3)):        # wrong total, wrong start, not monotone
        p = _gdn_problem(offsets=offs)
        assert lib.tt_gdn_tree_fwd(ctypes.byref(p), V, V, V, 1 << 30, None) == _lib.TT_E_ARG
    p = _gdn_problem()
    assert lib.tt_gdn_tree_fwd(ctypes.byref(p), None, V, V, 1 << 30, None) == _lib.TT_E_ARG
    assert lib.tt_gdn_tree_fwd(ctypes.byref(p), V, V, V, 64, None) == _lib.TT_E_WORKSPACE
    p = _gdn_problem(n_chunks=2)                      # fewer chunks than nodes
    assert lib.tt_gdn_tree_fwd(ctypes.byref(p), V, V, V, 1 << 30, None) == _lib.TT_E_ARG
    # per (chunk, v head): W, U [32 x 128], A, T [32 x 32], G [32] floats
    assert lib.tt_gdn_workspace_bytes(ctypes.byref(_gdn_problem())) == 5 * 32 * (2 * 32 * 128 + 2 * 32 * 32 + 2 * 32) * 4


def test_gdn_bwd_validation():
    lib = _lib.lib()
    V = ctypes.c_void_p(16)
    DO = _lib.TTTensor(16, 32 * 128, 128)
    p = _gdn_problem(node_child_off=16, node_child=16)
    per_chunk = (2 * 32 * 128 + 2 * 32 * 32 + 2 * 32) + 2 * 128 * 128 + 5 * 32 * 128 + 1
    want = (5 * 32 * per_chunk + 3 * 32 * 2 * 128 * 128) * 4
    assert lib.tt_gdn_bwd_workspace_bytes(ctypes.byref(p)) == want
    DQ = _lib.TTTensor(16, 16 * 128, 128)
    args = lambda ws_bytes, dq=DQ, dk=DQ, dv=DO, ds=None, di=None: (dq, dk, dv, V, V, ds, di, V, ws_bytes, None)
    assert lib.tt_gdn_tree_bwd(ctypes.byref(p), DO, *args(want - 4)) == _lib.TT_E_WORKSPACE
    assert lib.tt_gdn_tree_bwd(ctypes.byref(_gdn_problem()), DO, *args(want)) == _lib.TT_E_ARG   # no children CSR
    assert lib.tt_gdn_tree_bwd(ctypes.byref(p), _lib.TTTensor(18, 32 * 128, 128), *args(want)) == _lib.TT_E_ARG
    assert lib.tt_gdn_tree_bwd(ctypes.byref(p), _lib.TTTensor(16, 64, 128), *args(want)) == _lib.TT_E_ARG
    assert lib.tt_gdn_tree_bwd(ctypes.byref(p), DO, DQ, DQ, DO, ctypes.c_void_p(18), V, None, None, V, want,
                               None) == _lib.TT_E_ARG
    # the node-state gradient in and the initial-state gradient out: optional, 16-byte aligned
    assert lib.tt_gdn_tree_bwd(ctypes.byref(p), DO, *args(want - 4, ds=V, di=V)) == _lib.TT_E_WORKSPACE
    assert lib.tt_gdn_tree_bwd(ctypes.byref(p), DO, *args(want, ds=ctypes.c_void_p(20))) == _lib.TT_E_ARG
    assert lib.tt_gdn_tree_bwd(ctypes.byref(p), DO, *args(want, di=ctypes.c_void_p(24))) == _lib.TT_E_ARG
    # d_states_last_only: a flag (0: all node states' gradients, 1: the last node's alone)
    p.d_states_last_only = 2
    assert lib.tt_gdn_tree_bwd(ctypes.byref(p), DO, *args(want, ds=V)) == _lib.TT_E_ARG
    p.d_states_last_only = 0
    # dq/dk/dv: the row rules of q (a null, misaligned or short-strided output is refused) ...
    for bad in (_lib.TTTensor(None, 16 * 128, 128), _lib.TTTensor(24, 16 * 128, 128), _lib.TTTensor(16, 64, 128),
                _lib.TTTensor(16, 16 * 128, 100)):
        for i in range(3):
            outs = [DQ, DQ, DO]
            outs[i] = bad
            assert lib.tt_gdn_tree_bwd(ctypes.byref(p), DO, *args(want, *outs)) == _lib.TT_E_ARG
    # heads must be contiguous; rows at most 2^30 elements apart
    for i in range(3):
        outs = [DQ, DQ, DO]
        outs[i] = _lib.TTTensor(16, 64 * 128, 256)
        assert lib.tt_gdn_tree_bwd(ctypes.byref(p), DO, *args(want, *outs)) == _lib.TT_E_UNSUPPORTED
        outs[i] = _lib.TTTensor(16, (1 << 30) + 8, 128)
        assert lib.tt_gdn_tree_bwd(ctypes.byref(p), DO, *args(want, *outs)) == _lib.TT_E_ARG
    # ... and column blocks of one packed [T, (2 Hk + Hv) 128] row buffer pass them
    W = (2 * 16 + 32) * 128
    packed = (_lib.TTTensor(16, W, 128), _lib.TTTensor(16 + 16 * 128 * 2, W, 128),
              _lib.TTTensor(16 + 32 * 128 * 2, W, 128))
    assert lib.tt_gdn_tree_bwd(ctypes.byref(p), DO, *args(want - 4, *packed)) == _lib.TT_E_WORKSPACE
    assert lib.tt_gdn_tree_bwd(ctypes.byref(_gdn_problem(head_dim=64, node_child_off=16, node_child=16)), DO,
                               *args(want)) == _lib.TT_E_UNSUPPORTED


def test_gdn_saved_validation():
    """Forward that keeps what the backward needs, and the backward from it."""
    lib = _lib.lib()
    V = ctypes.c_void_p(16)
    DO = _lib.TTTensor(16, 32 * 128, 128)
    p = _gdn_problem(node_child_off=16, node_child=16)
    # per (chunk, v head): prep terms, initial state [128 x 128], V' [32 x 128]
    saved = 5 * 32 * ((2 * 32 * 128 + 2 * 32 * 32 + 2 * 32) + 128 * 128 + 32 * 128) * 4
    assert lib.tt_gdn_saved_bytes(ctypes.byref(p)) == saved
    # scratch: dS [128 x 128], dV', X, dW, dK~ [32 x 128], <S, dS> per chunk; dS at entry per node
    scratch = (5 * 32 * (128 * 128 + 4 * 32 * 128 + 1) + 3 * 32 * 128 * 128) * 4
    assert lib.tt_gdn_bwd_saved_workspace_bytes(ctypes.byref(p)) == scratch
    # the recomputing backward's workspace is the two plus the node states
    assert lib.tt_gdn_bwd_workspace_bytes(ctypes.byref(p)) == saved + scratch + 3 * 32 * 128 * 128 * 4
    assert lib.tt_gdn_tree_fwd_save(ctypes.byref(p), V, V, V, saved - 4, None) == _lib.TT_E_WORKSPACE
    assert lib.tt_gdn_tree_fwd_save(ctypes.byref(p), V, V, None, saved, None) == _lib.TT_E_ARG
    assert lib.tt_gdn_tree_fwd_save(ctypes.byref(p), V, V, ctypes.c_void_p(20), saved, None) == _lib.TT_E_ARG
    DQ = _lib.TTTensor(16, 16 * 128, 128)
    args = lambda sv, sb, wb: (DQ, DQ, DO, V, V, None, None, sv, sb, V, wb, None)
    assert lib.tt_gdn_tree_bwd_saved(ctypes.byref(p), DO, *args(V, saved - 4, scratch)) == _lib.TT_E_WORKSPACE
    assert lib.tt_gdn_tree_bwd_saved(ctypes.byref(p), DO, *args(V, saved, scratch - 4)) == _lib.TT_E_WORKSPACE
    assert lib.tt_gdn_tree_bwd_saved(ctypes.byref(p), DO, *args(None, saved, scratch)) == _lib.TT_E_ARG
    assert lib.tt_gdn_tree_bwd_saved(ctypes.byref(_gdn_problem()), DO, *args(V, saved, scratch)) == _lib.TT_E_ARG
    assert lib.tt_gdn_tree_bwd_saved(ctypes.byref(p), _lib.TTTensor(18, 32 * 128, 128),
                                     *args(V, saved, scratch)) == _lib.TT_E_ARG
    assert lib.tt_gdn_tree_bwd_saved(ctypes.byref(p), DO, _lib.TTTensor(16, 64, 128), DQ, DO, V, V, None, None, V,
                                     saved, V, scratch, None) == _lib.TT_E_ARG
    assert lib.tt_gdn_tree_bwd_saved(ctypes.byref(p), DO, DQ, DQ, DO, V, V, ctypes.c_void_p(20), None, V, saved, V,
                                     scratch, None) == _lib.TT_E_ARG


def _conv_problem(**kw):
    p = _lib.TTConvProblem(dtype=_lib.TT_DTYPE_BF16, n_tokens=10, n_channels=8, kernel_size=4, x=16,
                           x_stride_tok=8, weight=16, bias=None, tok_prev=16, tok_next_off=16, tok_next=16)
    for k, v in kw.items():
        setattr(p, k, v)
    return p


@pytest.mark.parametrize("field,value,code", [
    ("kernel_size", 5, _lib.TT_E_UNSUPPORTED),
    ("kernel_size", 0, _lib.TT_E_UNSUPPORTED),
    ("dtype", 9, _lib.TT_E_UNSUPPORTED),
    ("n_channels", 6, _lib.TT_E_ARG),            # not a multiple of 4
    ("x_stride_tok", 4, _lib.TT_E_ARG),          # rows overlap
    ("x", 12, _lib.TT_E_ARG),                    # misaligned for bf16x4
    ("tok_prev", None, _lib.TT_E_ARG),
])
def test_conv_validation(field, value, code):
    lib = _lib.lib()
    p = _conv_problem(**{field: value})
    assert lib.tt_tree_conv_fwd(ctypes.byref(p), ctypes.c_void_p(16), 8, None) == code


def test_conv_bwd_validation():
    lib = _lib.lib()
    V = ctypes.c_void_p(16)
    p = _conv_problem()
    # gp [T, C] + one partial block (K + 1 slots of C) in float32
    want = (10 * 8 + 1 * 5 * 8) * 4
    assert lib.tt_tree_conv_bwd_workspace_bytes(ctypes.byref(p)) == want
    assert lib.tt_tree_conv_bwd(ctypes.byref(p), V, 8, V, V, None, V, want - 4, None) == _lib.TT_E_WORKSPACE
    assert lib.tt_tree_conv_bwd(ctypes.byref(_conv_problem(tok_next=None)), V, 8, V, V, None, V, want,
                                None) == _lib.TT_E_ARG
    assert lib.tt_tree_conv_bwd(ctypes.byref(p), V, 4, V, V, None, V, want, None) == _lib.TT_E_ARG
    assert lib.tt_tree_conv_fwd(ctypes.byref(p), ctypes.c_void_p(20), 8, None) == _lib.TT_E_ARG


def _prologue_problem(**kw):
    p = _lib.TTPrologueProblem(dtype=_lib.TT_DTYPE_BF16, n_tokens=10, n_heads_q=32, n_heads_kv=8, head_dim=128,
                               eps_q=1e-6, eps_k=1e-6, q=_lib.TTTensor(16, 32 * 128, 128),
                               k=_lib.TTTensor(16, 8 * 128, 128), q_weight=16, k_weight=16, cos=16, sin=16,
                               cs_stride_tok=128)
    for k, v in kw.items():
        setattr(p, k, v)
    return p


@pytest.mark.parametrize("field,value,code", [
    ("head_dim", 64, _lib.TT_E_UNSUPPORTED),
    ("dtype", 3, _lib.TT_E_UNSUPPORTED),
    ("n_tokens", 0, _lib.TT_E_ARG),
    ("eps_q", float("nan"), _lib.TT_E_ARG),
    ("q", _lib.TTTensor(24, 32 * 128, 128), _lib.TT_E_ARG),      # misaligned rows
    ("k", _lib.TTTensor(16, 8 * 128, 100), _lib.TT_E_ARG),       # heads overlap
    ("cos", None, _lib.TT_E_ARG),
    ("cs_stride_tok", 64, _lib.TT_E_ARG),
])
def test_prologue_validation(field, value, code):
    lib = _lib.lib()
    p = _prologue_problem(**{field: value})
    assert lib.tt_qk_prologue_fwd(ctypes.byref(p), ctypes.c_void_p(16), ctypes.c_void_p(16), None) == code


def test_prologue_bwd_validation():
    lib = _lib.lib()
    V = ctypes.c_void_p(16)
    p = _prologue_problem()
    want = lib.tt_qk_prologue_bwd_workspace_bytes(ctypes.byref(p))
    assert want == 1024 * 2 * 128 * 4
    DQ, DK = _lib.TTTensor(16, 32 * 128, 128), _lib.TTTensor(16, 8 * 128, 128)
    assert lib.tt_qk_prologue_bwd(ctypes.byref(p), DQ, DK, V, V, V, V, V, want - 1, None) == _lib.TT_E_WORKSPACE
    assert lib.tt_qk_prologue_bwd(ctypes.byref(p), _lib.TTTensor(16, 64, 128), DK, V, V, V, V, V, want,
                                  None) == _lib.TT_E_ARG
    assert lib.tt_qk_prologue_bwd(ctypes.byref(p), DQ, DK, V, V, ctypes.c_void_p(18), V, V, want,
                                  None) == _lib.TT_E_ARG


def test_ce_rows_validation():
    lib = _lib.lib()
    V = ctypes.c_void_p(16)
    args = lambda **kw: dict(dict(dtype=_lib.TT_DTYPE_BF16, ld=1000, n=4, vocab=1000, ldg=1000), **kw)
    call = lambda a: lib.tt_ce_rows(a["dtype"], V, a["ld"], a["n"], a["vocab"], V, V, -100, V, V, a["ldg"], None)
    assert call(args(dtype=5)) == _lib.TT_E_UNSUPPORTED
    assert call(args(n=0)) == _lib.TT_E_ARG
    assert call(args(ld=999)) == _lib.TT_E_ARG          # shorter than a row
    assert call(args(ld=1004)) == _lib.TT_E_ARG         # rows not 16-byte aligned for bf16
    assert call(args(ldg=500)) == _lib.TT_E_ARG


def _det_slots(lens, par, bias=None, fn="tt_attn_det_slots"):
    import numpy as np
    nl, pa = np.asarray(lens, np.int32), np.asarray(par, np.int32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    out = ctypes.c_int64(-1)
    rc = getattr(_lib.lib(), fn)(nl.ctypes.data, pa.ctypes.data, len(nl),
                                 None if b is None else b.ctypes.data, 0 if b is None else len(b), ctypes.byref(out))
    return rc, out.value


def test_det_slots_match_visibility_windows():
    """tt_attn_det_slots and tt_attn_split_tiles (host only) against the dK/dV
    work-item rule applied to the oracle's dense visibility: per 128-key tile
    the union of its keys' visible queries is a range [lo, hi); a range longer
    than the window W (half the largest power of two <= n_q, clamped to
    [256, 4096]) is one work item per W-aligned window it touches (a split
    tile), others one item; the slots are the items beyond each tile's first.
    Forests with long nodes, with and without a gateway (bias 0 = seen by
    every query, -inf = by none)."""
    import numpy as np
    from oracle.tree_meta import mask_from_horizon, meta_closed_form
    from tree_training_amd import workloads
    rng = np.random.default_rng(5)
    for seed in range(6):
        lens, par = workloads.random_forest(seed, n_roots=(1, 2), max_depth=4, max_branch=3, node_len=(40, 700))
        T = sum(lens)
        mask = mask_from_horizon(meta_closed_form(lens, par)["horizon"])   # [query, key]
        for n_past in (0, 300):
            bias = None
            cols = mask
            if n_past:
                bias = np.where(rng.random(n_past) < 0.6, 0.0, -np.inf).astype(np.float32)
                cols = np.concatenate([np.repeat((bias == 0)[None, :], T, axis=0), mask], axis=1)
            half = (1 << (T.bit_length() - 1)) // 2
            W = min(4096, max(256, half))
            want = want_split = 0
            for kb in range(0, cols.shape[1], 128):
                rows = np.nonzero(cols[:, kb:kb + 128].any(axis=1))[0]
                if len(rows) == 0:
                    continue
                lo, hi = rows[0], rows[-1] + 1
                assert len(rows) == hi - lo        # one contiguous range
                if hi - lo > W:
                    want += (hi - 1) // W - lo // W
                    want_split += 1
            rc, got = _det_slots(lens, par, bias)
            assert rc == _lib.TT_OK
            assert got == want, (seed, n_past, got, want)
            rc, got = _det_slots(lens, par, bias, "tt_attn_split_tiles")
            assert rc == _lib.TT_OK
            assert got == want_split, (seed, n_past, got, want_split)
    # the workloads: far below the topology-free bound n_kb * floor((n_q - 1) / W)
    for (lens, par), n_past in ((workloads.agent_tree(0), 0), (workloads.agent_tree(0), 4096),
                                (workloads.rollout_tree(0), 0)):
        T = sum(lens)
        W = min(4096, max(256, (1 << (T.bit_length() - 1)) // 2))
        rc, got = _det_slots(lens, par, np.zeros(n_past) if n_past else None)
        assert rc == _lib.TT_OK and 0 < got < -(-(T + n_past) // 128) * ((T - 1) // W) / 2


@pytest.mark.parametrize("fn", ["tt_attn_det_slots", "tt_attn_split_tiles"])
def test_det_slots_rejects_bad_topology(fn):
    assert _det_slots([5, 0], [-1, 0], fn=fn)[0] == _lib.TT_E_ARG        # empty node
    assert _det_slots([5, 5], [-1, 1], fn=fn)[0] == _lib.TT_E_ARG        # parent not before the node
    assert _det_slots([5, 5], [-1, -2], fn=fn)[0] == _lib.TT_E_ARG
    assert _det_slots([], [], fn=fn)[0] == _lib.TT_E_ARG
    assert _det_slots([5, 5], [-1, 0], fn=fn)[1] == 0
