import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT / "moe-stream_amd", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: full-size shapes (seconds of CPU oracle work)")


def _gpu_visible() -> bool:
    # counting devices does not initialise HIP on this image; avoid torch here
    if os.environ.get("MOE_ROCM_FORCE_NO_GPU"):
        return False
    return any(Path("/dev").glob("dri/renderD*")) and Path("/dev/kfd").exists()


@pytest.fixture(scope="session")
def gpu_ctx():
    if not _gpu_visible():
        pytest.skip("no GPU visible")
    import moe_rocm as M

    ctx = M.Context(0)
    yield ctx
    ctx.close()
