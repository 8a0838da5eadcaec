"""Build the gfx950 C-ABI library ``_lib/libdels_mi355x.so`` in-tree with hipcc.

Usage: ``python dels-spec_amd/build.py`` (or ``build()`` from Python).  Always
recompiles; the output lands next to the package so it travels with the tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_DIR = os.path.join(PKG_DIR, "_lib")
LIB_NAME = "libdels_mi355x.so"
LIB_PATH = os.path.join(LIB_DIR, LIB_NAME)

SOURCES = ["capi.hip", "skinny_gemm.hip", "fused_argmax.hip", "fused_argmax_f32.hip", "fused_argmax_bf16.hip",
           "fused_argmax_f16.hip", "fused_argmax_tiled_f32.hip", "fused_argmax_tiled_bf16.hip",
           "fused_argmax_tiled_f16.hip", "lowrank_decode_f32.hip", "lowrank_decode_bf16.hip",
           "lowrank_decode_f16.hip", "pack.hip", "sample.hip", "domino_argmax.hip", "lm_head.hip",
           "rollout_resident.hip"]

# -packed-fp32-ops: never emit v_pk_{add,mul,fma}_f32 (kept off on this target).
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = os.path.join(rocm, "bin", "hipcc")
    return cand if os.path.exists(cand) else (shutil.which("hipcc") or "hipcc")


def build(verbose: bool = False, jobs: int | None = None, *, lib_path: str = LIB_PATH,
          extra_flags: tuple[str, ...] = (), link_flags: tuple[str, ...] = ()) -> str:
    """Compile every HIP source for gfx950 and link the shared library.

    ``extra_flags`` are added to every compile line and ``link_flags`` to the
    link line; with ``lib_path`` they give instrumented variants (the host-side
    sanitizer build of the tests) without touching the product library.
    """
    os.makedirs(os.path.dirname(lib_path), exist_ok=True)
    inc = ["-I", os.path.join(REPO_DIR, "include"), "-I", CSRC]
    tmp = tempfile.mkdtemp(prefix="dels_build_")
    try:
        objs = []
        procs = []
        for src in SOURCES:
            obj = os.path.join(tmp, src.replace(".hip", ".o"))
            cmd = [hipcc(), *HIP_FLAGS, *extra_flags, *inc, "-c", os.path.join(CSRC, src), "-o", obj]
            if verbose:
                print(" ".join(cmd), flush=True)
            procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
            objs.append(obj)
        failed = []
        for src, p in procs:
            out, _ = p.communicate()
            text = out.decode(errors="replace")
            # hipcc's host pass does not know the gfx feature flag; that note is harmless.
            text = "\n".join(l for l in text.splitlines() if "packed-fp32-ops" not in l)
            if p.returncode != 0:
                failed.append(src)
                sys.stderr.write(f"--- hipcc failed on {src} ---\n{text}\n")
            elif verbose and text.strip():
                sys.stderr.write(text + "\n")
        if failed:
            raise RuntimeError(f"hipcc failed on {failed}")
        tmp_lib = lib_path + ".tmp"
        cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *link_flags, "-o", tmp_lib, *objs]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        os.replace(tmp_lib, lib_path)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return lib_path


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
