"""The library the GPU tests load is the one built from the sources beside it: its version string carries the
hash of csrc/ and include/a8attn.h (ensure_built() rebuilds a stale library where a compiler is at hand)."""
from __future__ import annotations

import importlib.util
import os

import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_gpu_run_loads_the_current_library(a8):
    spec = importlib.util.spec_from_file_location("_a8_bl", os.path.join(ROOT, "audio8-turbo-engine_amd", "build_lib.py"))
    bl = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bl)
    ver = a8.load_library().a8_version().decode()
    print(f"case: library {ver}", flush=True)
    assert ver.endswith("src:" + bl.source_hash()), (ver, bl.source_hash())
