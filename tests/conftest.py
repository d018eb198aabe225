import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _ensure_built():
    """Tests load what is built; only if nothing is, build it (without forcing)."""
    if not (ROOT / "l3m_amd" / "libl3m_hip.so").exists():
        subprocess.run(["make", "-s", "-C", str(ROOT / "l3m_amd" / "csrc")], check=True)
    if not (ROOT / "oracle" / "liboracle.so").exists():
        subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "all"], check=True)


_ensure_built()


@pytest.fixture(scope="session")
def oracle():
    from oracle.oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def reference():
    from oracle.oracle import Reference
    if not Reference.available():
        pytest.skip("oracle/_ref (the reference built from source) is not present")
    return Reference()


@pytest.fixture(scope="session")
def dev():
    import l3m_amd
    return l3m_amd.Device()


@pytest.fixture(scope="session")
def golden():
    return json.loads((GOLDEN / "decode.json").read_text())


class ModelCache:
    """Synthetic models written once per session: key (config, dtype, seed, extra kwargs)."""

    def __init__(self, root):
        self.root, self.paths = root, {}

    def get(self, cfg, dtype=None, seed=1, **kw):
        import l3m_amd as A
        name = cfg if isinstance(cfg, str) else cfg.name
        key = (name, dtype, seed, tuple(sorted(kw.items())))
        if key not in self.paths:
            p = self.root / f"{name}-{dtype}-{seed}-{len(self.paths)}.l3m"
            self.paths[key] = A.write_model(p, cfg, dtype=dtype, seed=seed, **kw)
        return self.paths[key]


@pytest.fixture(scope="session")
def models(tmp_path_factory):
    return ModelCache(tmp_path_factory.mktemp("models"))


@pytest.fixture(scope="session")
def dev_free():
    """Host-side packing helpers of l3m_amd.Device, without initialising a GPU."""
    import l3m_amd
    d = l3m_amd.Device.__new__(l3m_amd.Device)
    d.lib = l3m_amd.lib()
    return d
