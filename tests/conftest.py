import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref_oracle():
    from oracle import RefOracle, ref_available
    if not ref_available():
        pytest.skip("oracle/_ref not built (needs /root/reference)")
    return RefOracle()


@pytest.fixture(scope="session")
def cfg1_stage():
    """cfg1 inputs prepared by the product host code (groups, reorder, LNG)."""
    import filtervectorcode_refactor_amd as F
    from filtervectorcode_refactor_amd import datasets as D
    X, lp, li = D.generate(D.CONFIGS["cfg1"])
    st = F.UngBuildStage()
    st.prepare_inputs(X, lp, li)
    return st


def golden_path(name):
    return os.path.join(ROOT, "tests", "golden", name)


def load_golden(name):
    p = golden_path(name)
    if not os.path.exists(p):
        pytest.skip(f"golden fixture {name} missing")
    with np.load(p, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}
