"""Shared fixtures. Tests marked `gpu` need a HIP device and call the kernels through the C ABI;
everything else runs on the CPU (oracle pinning, host logic, library exports)."""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import __graft_entry__  # noqa: E402

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X); parity tests through the C ABI")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no HIP device in this process")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


@pytest.fixture(scope="session")
def a8():
    __graft_entry__.ensure_built()
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def ref():
    from oracle import attn_ref
    return attn_ref


@pytest.fixture(scope="session")
def dev():
    return torch.device("cuda:0")


def golden(name):
    with np.load(os.path.join(GOLDEN, name)) as z:
        return {k: z[k] for k in z.files}


def bf16_from_bits(a):
    """uint16 bf16 bit patterns (numpy) -> torch bf16 tensor."""
    return torch.from_numpy(np.ascontiguousarray(a).astype(np.int16)).view(torch.bfloat16)


def bits_of(t):
    """torch bf16 tensor -> uint16 numpy bit patterns."""
    return t.contiguous().view(torch.int16).numpy().astype(np.uint16)


def randn_bf16(g, *shape, std=1.0):
    return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16)
