import os
import pathlib
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "ltx-zml_amd"))
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def block0():
    """Synthetic block 0: Student-t(3) x 0.02 weights, int8-g128 qkv + ff (the
    reference recipe), f32 scales."""
    from ltx_amd import synth
    return synth.make_block(0, seed=1, dist="t3")


@pytest.fixture(scope="session")
def block0_out():
    """Same block with the out-projections quantised too (every large GEMM int8)."""
    from ltx_amd import synth
    return synth.make_block(0, seed=1, dist="t3", classes=("qkv", "ff", "out"))


@pytest.fixture(scope="session")
def block0_w16():
    """The same block unquantised (every projection in its bf16 weights): the
    recipe of Block.wBlockOut (ltx/block.zig:351-353), the reference's
    production caller (ltx/e2e_prod.zig:382-399)."""
    from ltx_amd import synth
    return synth.make_block(0, seed=1, dist="t3", classes=())


@pytest.fixture(scope="session")
def ctx():
    import torch
    from ltx_amd import runtime
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    c = runtime.Context(0)
    yield c
    c.close()


def say(msg: str) -> None:
    """Progress line naming the case before each GPU step."""
    print(msg, flush=True)
    sys.stdout.flush()
