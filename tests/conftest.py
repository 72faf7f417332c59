import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libmarian_hip.so)")


@pytest.fixture(scope="session")
def pkg():
    import __graft_entry__ as ge

    return ge.load_package()


@pytest.fixture(scope="session")
def orc():
    import __graft_entry__ as ge

    return ge.load_oracle()


@pytest.fixture(scope="session")
def kats():
    import json

    return json.loads((ROOT / "tests" / "golden" / "reference_kats.json").read_text())


@pytest.fixture(scope="session")
def small_model(pkg):
    geom = pkg.Geometry(vocab=2048, dim=512, heads=8, ffn_dim=2048, encoder_layers=2,
                        decoder_layers=2)
    return pkg.seeded_model(seed=7, geometry=geom)


@pytest.fixture(scope="session")
def full_model(pkg):
    return pkg.seeded_model()
