"""Shared fixtures. GPU tests are marked @pytest.mark.gpu and call the product through its C ABI
(miso_amd/lib/libmiso_attn.so, via miso_amd.attention); the CPU oracle (oracle/) is the checker.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def O():
    from oracle import oracle
    return oracle


@pytest.fixture(scope="session")
def torch_mod():
    import torch
    return torch


@pytest.fixture(scope="session")
def attn(torch_mod):
    """The product's operator module; the HIP library must load (no fallback exists)."""
    if not torch_mod.cuda.is_available():
        pytest.fail("GPU test collected without a GPU")
    from miso_amd import attention
    attention._lib.load()
    return attention


@pytest.fixture(scope="session")
def ref_kernels(O, attn):
    """The reference's kernels built from its sources (oracle/_ref), if that library exists."""
    return O.ref_kernels()


def to_dev(torch, a: np.ndarray):
    """numpy -> device tensor; uint16 (binary16 bits) becomes a float16 tensor with those bits."""
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).cuda().view(torch.float16)
    if a.dtype == np.uint64:
        return torch.from_numpy(a.view(np.int64).copy()).cuda()
    if a.dtype == np.uint32:
        return torch.from_numpy(a.astype(np.int32)).cuda()
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def to_host(t) -> np.ndarray:
    import torch
    t = t.detach()
    if t.dtype == torch.float16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


# The reference's own accuracy gate for its decode and prefill kernels: per-(token, head) relative
# L2 error against the FP64 host reference <= 1e-5 (tests/test_attn_splitk.hip:174, :267). The
# f32-arithmetic decode paths are held to it on top of the elementwise north-star tolerance.
REF_REL_L2 = 1e-5


def report(name: str, stats: dict) -> None:
    print(f"[{name}] max_abs={stats['max_abs']:.3e} max_rel={stats['max_rel']:.3e} "
          f"rel_l2={stats['rel_l2']:.3e} rel_l2_head={stats['rel_l2_head']:.3e} "
          f"bad={stats['n_bad']}", flush=True)
