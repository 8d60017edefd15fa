import os
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
for p in (HERE, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


_layers = {}


@pytest.fixture(scope="session")
def layer_cache():
    """Seeded synthetic layers are expensive to build; share them per session."""
    import zzref

    def get(kind, seed=1, **kw):
        key = (kind, seed, tuple(sorted(kw.items())))
        if key not in _layers:
            _layers[key] = zzref.make_layer(kind, seed=seed, **kw)
        return _layers[key]

    return get
