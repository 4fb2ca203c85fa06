"""Shared pytest setup.

Markers: `gpu` tests need an MI355X (gfx950) and the built libckh.so; everything else
runs on the CPU.  The product package lives in comfy-kitchen_amd/ and is imported as
`comfy_kitchen`; the CPU oracle (test infrastructure) is the top-level `oracle` package.
"""
import sys
from pathlib import Path

import pytest
import torch

REPO = Path(__file__).resolve().parent.parent
for p in (REPO / "comfy-kitchen_amd", REPO):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running test")


def gpu_ready() -> tuple[bool, str]:
    import comfy_kitchen as ck

    info = ck.list_backends().get("hip", {})
    if not info.get("available"):
        return False, info.get("unavailable_reason") or "hip backend not registered"
    return True, ""


@pytest.fixture
def seed():
    torch.manual_seed(42)
    yield


@pytest.fixture(scope="session")
def hip():
    """Require the hip backend; on a GPU box a missing/broken library is a failure, not a skip."""
    ok, why = gpu_ready()
    if not ok:
        if torch.cuda.is_available():
            pytest.fail(f"GPU present but hip backend unavailable: {why}")
        pytest.skip(why)
    import comfy_kitchen.backends.hip as hb

    return hb


@pytest.fixture(scope="session")
def scalar_ref():
    from oracle import build_ref

    return build_ref.load()


@pytest.fixture(scope="session")
def dev():
    return torch.device("cuda", 0)


def bits(t: torch.Tensor) -> torch.Tensor:
    """Raw bytes/halves of a tensor as an integer tensor on the CPU (for bit-exact compares)."""
    t = t.detach().cpu().contiguous()
    if t.element_size() == 1:
        return t.view(torch.uint8)
    if t.element_size() == 2:
        return t.view(torch.int16)
    return t.view(torch.int32)
