"""Builds the gfx950 HIP library behind the C ABI (include/a8attn.h) into this package, in-tree.

`python build_lib.py` (or `__graft_entry__.build()`) compiles every source in csrc/ with hipcc for
gfx950 only and links one shared library, `liba8attn.so`, next to this file. The library links the
HIP runtime by soname (libamdhip64.so.7), so inside a process that has imported torch it binds to
the runtime torch already loaded and shares its streams and graphs.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "liba8attn.so")
SOURCES = ["capi.hip", "store.hip", "decode.hip", "decode_stream.hip", "decode_flat.hip", "prefill.hip",
           "prefix_copy.hip", "layer_ops.hip", "conv.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # packed fp32 VALU ops are kept out of every kernel (the compiler would otherwise form them
    # from float2-shaped code); this is a device-side feature flag, the host pass ignores it.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = os.path.join(rocm, "bin", "hipcc")
    return path if os.path.exists(path) else "hipcc"


def build(verbose: bool = False, extra_flags=None) -> str:
    """Compile csrc/*.hip for gfx950 into liba8attn.so (always rebuilds). Returns the library path."""
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    tmp = LIB + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, *(extra_flags or []), *srcs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass warns about the device-only feature flag; anything else is worth showing
    noise = "'-packed-fp32-ops' is not a recognized feature for this target (ignoring feature)"
    msgs = [ln for ln in (res.stdout + res.stderr).splitlines() if noise not in ln and ln.strip()]
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(msgs))
    if msgs and verbose:
        print("\n".join(msgs))
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
