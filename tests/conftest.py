"""Shared fixtures: the product binding (turkce-llm_amd/trlm.py, loaded by
path because the package directory is not an identifier) and the oracle."""
import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path through the C ABI)")


def load_trlm():
    name = "trlm_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, os.path.join(ROOT, "turkce-llm_amd", "trlm.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def parity_report(name, rows, header="tensor  max|got-want|  max|want|  ratio"):
    """Per-tensor max-abs errors of a parity test: printed, and written to
    $TRLM_PARITY_REPORT/<name>.txt when that directory is set."""
    lines = [header] + ["%-16s %.3e  %.3e  %.2e" % (n, e, m, e / (m + 1e-30)) for n, e, m in rows]
    print("\n".join(["[%s]" % name] + lines))
    out = os.environ.get("TRLM_PARITY_REPORT")
    if out:
        os.makedirs(out, exist_ok=True)
        with open(os.path.join(out, name + ".txt"), "w") as fh:
            fh.write("\n".join(lines) + "\n")


@pytest.fixture(scope="session")
def trlm():
    return load_trlm()


@pytest.fixture(scope="session")
def orc():
    import oracle
    return oracle
