import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


# Parity figures that tests report (identical-id prefixes, worst errors over
# long decodes): printed in the terminal summary, which `pytest -q` keeps, and
# written as JSON lines to $LSSM_PARITY_RECORD when that is set.
RECORDS = []


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def pytest_terminal_summary(terminalreporter):
    if not RECORDS:
        return
    import json
    terminalreporter.write_sep("-", "parity records")
    for r in RECORDS:
        terminalreporter.write_line(json.dumps(r, sort_keys=True, default=float))
    path = os.environ.get("LSSM_PARITY_RECORD")
    if path:
        with open(path, "a") as f:
            for r in RECORDS:
                f.write(json.dumps(r, sort_keys=True, default=float) + "\n")


@pytest.fixture(scope="session")
def progress(request):
    """say(msg): print a progress line past pytest's output capture, so that a
    test which runs for minutes shows on the console that it is advancing."""
    capman = request.config.pluginmanager.getplugin("capturemanager")

    def say(msg):
        if capman is None:
            print(msg, flush=True)
            return
        with capman.global_and_fixture_disabled():
            print(msg, flush=True)
    return say


@pytest.fixture
def parity_record():
    """record(name, **figures): keep a test's parity figures for the summary."""
    def record(name, **fig):
        RECORDS.append(dict(test=name, **fig))
        print(f"[parity] {name}: {fig}", flush=True)
    return record


@pytest.fixture(scope="session")
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


@pytest.fixture(scope="session")
def ctx(torch_cuda):
    import lite_ssm_amd as L
    # a dedicated (default-priority) stream shared by torch copies and the
    # library, so ordering is implicit and HIP-graph capture is legal
    s = torch_cuda.cuda.Stream()
    torch_cuda.cuda.set_stream(s)
    c = L.Ctx(stream=s.cuda_stream)
    yield c
    c.close()


@pytest.fixture
def rng():
    return np.random.default_rng(1234)


@pytest.fixture(autouse=True)
def _keep_device_copies():
    yield
    try:
        import gpu_util
        gpu_util.KEEP.clear()
    except ImportError:
        pass
