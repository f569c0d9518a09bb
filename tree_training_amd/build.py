"""Builds the in-tree HIP library ``tree_training_amd/lib/libtree_attn.so`` for gfx950.

Run ``python -m tree_training_amd.build`` (or ``__graft_entry__.build()``). The
library is compiled from the sources in ``csrc/`` with hipcc, one object per
translation unit, then linked as a shared object exposing the C ABI declared in
``include/tree_attn.h``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
LIBDIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIBDIR, "libtree_attn.so")
SOURCES = ["tt_meta.hip", "tt_attn_fwd_bf16.hip", "tt_attn_bwd_bf16.hip", "tt_attn_f32.hip", "tt_gdn.hip", "tt_gdn_trunc.hip",
           "tt_conv.hip", "tt_prologue.hip", "tt_ce.hip",
           "tt_api.hip", "tt_noalloc.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17",
    "-munsafe-fp-atomics",
    # packed fp32 VALU ops are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = os.path.join(rocm, "bin", "hipcc")
    return cand if os.path.exists(cand) else (shutil.which("hipcc") or cand)


# Per-source flags. The bf16 forward never produces or consumes NaN (masked
# scores are -inf and every exp2/max/sum on them is guarded), so it is built
# without NaN semantics and with IEEE mode off: its row max then needs no
# operand canonicalisation (v_max3_f32 straight on MFMA results).
SOURCE_FLAGS = {"tt_attn_fwd_bf16.hip": ["-fno-honor-nans", "-mno-amdgpu-ieee"]}


def _compile(src: str, obj: str, extra):
    cmd = [hipcc(), *HIPCC_FLAGS, *SOURCE_FLAGS.get(src, []), *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return r.stderr


def build(verbose: bool = False, extra=(), out: str = LIB) -> str:
    """Compiles every HIP source and links the shared library; returns its path."""
    objdir = os.path.join(PKG, "_build" if out == LIB else "_build_alt")
    os.makedirs(objdir, exist_ok=True)
    os.makedirs(os.path.dirname(out), exist_ok=True)
    objs = [os.path.join(objdir, s.replace(".hip", ".o")) for s in SOURCES]
    with ThreadPoolExecutor(max_workers=min(6, len(SOURCES))) as ex:
        logs = list(ex.map(lambda so: _compile(so[0], so[1], list(extra)), zip(SOURCES, objs)))
    if verbose:
        for s, log in zip(SOURCES, logs):
            print(f"[{s}]\n{log}")
    tmp = out + ".tmp"
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    args = sys.argv[1:]
    out = LIB
    if "--out" in args:
        i = args.index("--out")
        out = os.path.abspath(args[i + 1])
        args = args[:i] + args[i + 2:]
    print(build(verbose=True, extra=args, out=out))
