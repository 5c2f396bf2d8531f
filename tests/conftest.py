import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built library")


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


class Golden:
    """Access to one golden npz: golden.case(name) -> dict of arrays."""

    def __init__(self, group):
        self.data = np.load(os.path.join(GOLDEN, f"{group}.npz"), allow_pickle=False)
        with open(os.path.join(GOLDEN, "manifest.json")) as fh:
            self.meta = json.load(fh).get(group, {})

    def case(self, name):
        pre = name + "/"
        return {k[len(pre):]: self.data[k] for k in self.data.files if k.startswith(pre)}

    def names(self):
        return sorted({k.split("/")[0] for k in self.data.files})


@pytest.fixture(scope="session")
def golden():
    return Golden


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    if not os.path.exists(O.LIB):
        O.build()
    return O


TORCH_DT = {"f32": "float32", "f16": "float16", "bf16": "bfloat16"}


def to_torch(storage, dtype, device="cuda"):
    """Golden storage array (bf16 as uint16 bits) -> torch tensor on device."""
    import torch
    a = np.ascontiguousarray(storage)
    if dtype == "bf16":
        t = torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
    else:
        t = torch.from_numpy(a.copy())
    return t.to(device)


def to_values(t):
    """torch tensor -> float32 numpy values (exact for f16 / bf16)."""
    return t.detach().float().cpu().numpy()


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


def torch_dtype(name):
    import torch
    return getattr(torch, TORCH_DT[name])


def seed_of(*parts):
    """Deterministic 32-bit seed from a test's parameters."""
    import zlib
    return zlib.crc32(repr(parts).encode())
