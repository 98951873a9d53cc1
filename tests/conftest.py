import os
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


@pytest.fixture(scope="session")
def vqx():
    import __graft_entry__

    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def golden():
    return np.load(os.path.join(ROOT, "tests", "golden", "tables.npz"))


def bits(t):
    """Raw bit patterns of a float tensor/array as unsigned ints (numpy)."""
    if isinstance(t, torch.Tensor):
        t = t.detach().cpu()
        if t.dtype == torch.bfloat16:
            return t.view(torch.int16).numpy().view(np.uint16)
        if t.dtype == torch.float16:
            return t.view(torch.int16).numpy().view(np.uint16)
        return t.view(torch.int32).numpy().view(np.uint32)
    a = np.asarray(t)
    return a.view(np.uint32) if a.dtype == np.float32 else a.view(np.uint16)


def assert_bitexact(got, want, what=""):
    """Bit-exact equality, every NaN counting as equal to every NaN."""
    g = got.detach().cpu().float() if isinstance(got, torch.Tensor) else torch.from_numpy(np.asarray(got)).float()
    w = want.detach().cpu().float() if isinstance(want, torch.Tensor) else torch.from_numpy(np.asarray(want)).float()
    assert g.shape == w.shape, f"{what}: shape {tuple(g.shape)} vs {tuple(w.shape)}"
    gb = g.view(torch.int32)
    wb = w.view(torch.int32)
    ok = (gb == wb) | (torch.isnan(g) & torch.isnan(w))
    if not bool(ok.all()):
        bad = (~ok).nonzero()
        i = tuple(bad[0].tolist())
        raise AssertionError(f"{what}: {int((~ok).sum())} of {ok.numel()} differ; first at {i}: "
                             f"got {g[i].item()!r} ({hex(gb[i].item() & 0xFFFFFFFF)}) "
                             f"want {w[i].item()!r} ({hex(wb[i].item() & 0xFFFFFFFF)})")
