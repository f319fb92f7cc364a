"""Shared fixtures.  `-m gpu` selects the tests that need an MI355X."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (run with -m gpu)")


@pytest.fixture(scope="session")
def oracle():
    from oracle.bindings import oracle as load
    return load()


@pytest.fixture(scope="session")
def golden_kernels():
    import numpy as np
    with np.load(ROOT / "tests" / "golden" / "kernels.npz", allow_pickle=False) as data:
        return {k: data[k] for k in data.files}


@pytest.fixture(scope="session")
def golden_decoders():
    import json
    import numpy as np
    with np.load(ROOT / "tests" / "golden" / "decoders.npz", allow_pickle=False) as data:
        arrays = {k: data[k] for k in data.files}
    meta = json.loads((ROOT / "tests" / "golden" / "decoders.json").read_text())
    return arrays, meta


@pytest.fixture(scope="session")
def artifacts(tmp_path_factory):
    """Reduced synthetic artifacts of every family (same specs as the golden vectors)."""
    from leaf_amd.artifact import write_artifact
    from tests.golden.make_golden import decoder_spec, DECODER_CASES
    root = tmp_path_factory.mktemp("artifacts")
    out = {}
    for family in DECODER_CASES:
        path = root / f"{family}.leaf"
        write_artifact(path, decoder_spec(family), seed=101)
        out[family] = path
    return out


@pytest.fixture(scope="session")
def full_artifacts(tmp_path_factory):
    """The benchmark configurations' full-size synthetic artifacts, written on first use."""
    from leaf_amd import models
    from leaf_amd.artifact import write_artifact
    from tests.golden.make_golden import FULL_ARTIFACT_SEED
    root = tmp_path_factory.mktemp("full")
    cache = {}

    def get(family):
        if family not in cache:
            path = root / f"{family}.leaf"
            write_artifact(path, models.PRESETS[family](), seed=FULL_ARTIFACT_SEED)
            cache[family] = path
        return cache[family]
    return get


@pytest.fixture(scope="session")
def golden_features():
    import json
    import numpy as np
    with np.load(ROOT / "tests" / "golden" / "features.npz", allow_pickle=False) as data:
        arrays = {k: data[k] for k in data.files}
    meta = json.loads((ROOT / "tests" / "golden" / "features.json").read_text())
    return arrays, meta


@pytest.fixture(scope="session")
def feature_artifacts(tmp_path_factory, golden_features):
    """Reduced artifacts of the operator and storage features, written on first use."""
    from leaf_amd.artifact import write_artifact
    from tests.golden.make_golden import feature_spec
    root = tmp_path_factory.mktemp("features")
    _, meta = golden_features
    cache = {}

    def get(name):
        if name not in cache:
            path = root / f"{name}.leaf"
            write_artifact(path, feature_spec(name, meta[name]["eos_tokens"]), seed=meta[name]["seed"])
            cache[name] = path
        return cache[name]
    return get
