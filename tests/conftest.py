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
def knob_gemm(gemm):
    """(tile, splits) → a context on cuda:0 created with SQ8_TILE = tile and SQ8_SPLITS = splits (None: unset;
    the library reads its knobs once, when a context is created). Contexts are kept per pair."""
    import siliconed_amd as sq
    made = {}

    def get(tile=None, splits=None):
        key = (tile, splits)
        if key not in made:
            env = {"SQ8_TILE": tile, "SQ8_SPLITS": None if splits is None else str(splits)}
            old = {name: os.environ.get(name) for name in env}
            try:
                for name, value in env.items():
                    if value is None:
                        os.environ.pop(name, None)
                    else:
                        os.environ[name] = value
                made[key] = sq.TensorGEMM.make(0)
            finally:
                for name, value in old.items():
                    if value is None:
                        os.environ.pop(name, None)
                    else:
                        os.environ[name] = value
        return made[key]

    return get


@pytest.fixture(scope="session")
def tile_gemm(knob_gemm):
    """knob → a context on cuda:0 created with SQ8_TILE = knob: the product on that forced weight-direct tile."""
    return lambda knob: knob_gemm(knob, None)
