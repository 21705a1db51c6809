import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu")
    config.addinivalue_line("markers", "slow: long-running GPU case (grid / stress)")


@pytest.fixture(scope="session")
def oracle_mod():
    import oracle

    oracle.build()
    return oracle


@pytest.fixture(scope="session")
def fa_lib():
    """The HIP product library, built in-tree if absent (hipcc cross-compiles)."""
    import cuda_fused_attention_amd as fa

    if not os.path.exists(fa.LIB_PATH):
        from cuda_fused_attention_amd import _build

        _build.build()
    fa.lib()
    return fa
