import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
for path in (ROOT, ROOT / "tests"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))

import nvs_amd  # noqa: E402,F401  (registers the package directory under its import name)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm device) and the built libnvs_amd.so")


@pytest.fixture(scope="session")
def device():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    from nvs_amd import _lib
    _lib.load()  # the HIP path must be the one under test: a missing library fails loudly here
    return torch.device("cuda", torch.cuda.current_device())


def log_case(name: str) -> None:
    """Name the case on stdout before a GPU step, so a run that dies mid-test still says which one it was."""
    print(f"[case] {name}", flush=True)
