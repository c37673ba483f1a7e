import sys
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
sys.path.insert(0, str(HERE.parent))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; parity tests through the C ABI")
    config.addinivalue_line("markers", "slow: full-size shapes (seconds of oracle time)")


@pytest.fixture(scope="session")
def gpu():
    """The GPU, made current through the library's own device call. GPU tests never skip
    silently: without a device they fail."""
    import torch

    from tensorlisp_amd import native

    assert torch.cuda.is_available(), "a gpu-marked test ran without a GPU"
    props = native.device_props(0)
    print(f"\n[gpu] {props['name']} {props['arch']} CUs={props['compute_units']} "
          f"LDS={props['lds_bytes']} clock={props['clock_khz']}kHz", flush=True)
    return props
