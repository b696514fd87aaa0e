import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
PKG = REPO / "memory-aware-inference_amd"
for p in (str(PKG), str(REPO / "tests"), str(REPO)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _ensure_built():
    import oracle_lib
    if not oracle_lib.ORACLE_SO.exists():
        oracle_lib.build()
    lib = PKG / "si_hip" / "libsi_hip.so"
    if not lib.exists():
        sys.path.insert(0, str(PKG))
        import build as pkg_build
        pkg_build.build()


_ensure_built()


@pytest.fixture(scope="session")
def hip_ctx():
    import si_hip
    ctx = si_hip.HipContext(0)
    yield ctx
    ctx.close()
