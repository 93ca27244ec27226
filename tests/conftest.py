import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "mini-inference_amd", ROOT / "tests" / "golden"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

import torch  # noqa: E402

HAS_GPU = torch.cuda.is_available()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built libmipaged.so")


@pytest.fixture(scope="session")
def gpu():
    """The device the kernels run on; fails loudly (no fallback) if the library is not built."""
    if not HAS_GPU:
        pytest.skip("no ROCm GPU in this environment")
    from engine import _native

    _native.load()  # raises NativeLibraryMissing
    return torch.device("cuda", 0)


def announce(msg: str) -> None:
    """Print and flush the case name before a GPU step, so a fault can be traced to it."""
    print(f"[case] {msg}", file=sys.__stdout__, flush=True)
