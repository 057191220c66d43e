import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950); runs the HIP library through its C ABI")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def gemm():
    """The library's context on cuda:0 (GPU tests only)."""
    import torch
    import siliconed_amd as sq
    assert torch.cuda.is_available(), "a gpu-marked test ran without a GPU"
    ctx = sq.TensorGEMM.make(0)
    assert ctx is not None, "cuda:0 is not a gfx950"
    return ctx


@pytest.fixture(scope="session")
def tile_gemm(gemm):
    """knob → a context on cuda:0 created with SQ8_TILE = knob (the library reads its tile knobs once, when
    a context is created): the product on that forced weight-direct tile. Contexts are kept per knob."""
    import siliconed_amd as sq
    made = {}

    def get(knob: str):
        if knob not in made:
            old = os.environ.get("SQ8_TILE")
            os.environ["SQ8_TILE"] = knob
            try:
                made[knob] = sq.TensorGEMM.make(0)
            finally:
                if old is None:
                    os.environ.pop("SQ8_TILE", None)
                else:
                    os.environ["SQ8_TILE"] = old
        return made[knob]

    return get
