"""Builds the gfx950 HIP library behind the C ABI (include/a8attn.h) into this package, in-tree.

`python build_lib.py` (or `__graft_entry__.build()`) compiles every source in csrc/ with hipcc for
gfx950 only (objects in _build/, one compiler process per source) and links one shared library, `liba8attn.so`, next to this file. The library links the
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
SOURCES = ["capi.hip", "store.hip", "decode.hip", "decode_stream.hip", "decode_rows.hip", "decode_flat.hip", "prefill.hip",
           "prefill128.hip", "attn_cols.hip",
           "prefix_copy.hip", "layer_ops.hip", "gemm.hip", "decode_f32q.hip", "conv.hip"]

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


# Per-source flags. The decode kernels hold their softmax accumulators in VGPRs: at the register pressure of the
# whole-row kernel the compiler otherwise puts the MFMA accumulators in AGPRs and copies them to VGPRs and back
# around the softmax rescale and the merge (C3 fused store + decode measured 36.51 -> 36.18 us per layer on one
# box with the VGPR form).
SOURCE_FLAGS = {src: ["-mllvm", "-amdgpu-mfma-vgpr-form"]
                for src in ("decode.hip", "decode_stream.hip", "decode_rows.hip", "decode_flat.hip")}


def source_hash() -> str:
    """A short hash of every source the library is built from (csrc/ and include/a8attn.h); the build bakes it
    into a8_version(), so a library older than its sources can be told apart."""
    import hashlib
    h = hashlib.sha1()
    inc = os.path.join(os.path.dirname(HERE), "include", "a8attn.h")
    for p in sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC)) + [inc]:
        if os.path.isfile(p):
            h.update(os.path.basename(p).encode())
            with open(p, "rb") as f:
                h.update(f.read())
    return h.hexdigest()[:12]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = os.path.join(rocm, "bin", "hipcc")
    return path if os.path.exists(path) else "hipcc"


def _run(cmd):
    res = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass warns about the device-only feature flag; anything else is worth showing
    noise = "'-packed-fp32-ops' is not a recognized feature for this target (ignoring feature)"
    msgs = [ln for ln in (res.stdout + res.stderr).splitlines() if noise not in ln and ln.strip()]
    return res.returncode, msgs


def build(verbose: bool = False, extra_flags=None, jobs=None) -> str:
    """Compile csrc/*.hip for gfx950 (one hipcc per source, in parallel) and link liba8attn.so (always
    rebuilds). Returns the library path."""
    from concurrent.futures import ThreadPoolExecutor

    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    flags = [f for f in HIPCC_FLAGS if f != "-shared"] + list(extra_flags or []) + [f'-DA8_SRC_HASH="{source_hash()}"']
    jobs = jobs or max(1, min(len(SOURCES), os.cpu_count() or 1, 16))

    def compile_one(src):
        obj = os.path.join(objdir, os.path.splitext(src)[0] + ".o")
        cmd = [hipcc(), *flags, *SOURCE_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        return obj, _run(cmd)

    with ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(compile_one, SOURCES))
    objs, errs = [], []
    for obj, (rc, msgs) in results:
        objs.append(obj)
        if rc != 0:
            errs += msgs
        elif msgs and verbose:
            print("\n".join(msgs))
    if errs:
        raise RuntimeError("hipcc failed:\n" + "\n".join(errs))
    tmp = LIB + ".tmp"
    rc, msgs = _run([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp])
    if rc != 0:
        raise RuntimeError("link failed:\n" + "\n".join(msgs))
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
