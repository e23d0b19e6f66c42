import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm device) and the built HIP library")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda:0")


def seeded(seed: int):
    import torch

    g = torch.Generator()
    g.manual_seed(seed)
    return g


# Near-tie / mismatch counts recorded by the parity tests; printed in the
# terminal summary (visible under -q) and written to gpurun_out/ when present.
PARITY_RECORDS: list = []


@pytest.fixture(scope="session")
def parity_report():
    return PARITY_RECORDS


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    if not PARITY_RECORDS:
        return
    import json

    terminalreporter.section("index parity vs the reference (disagreements by class)")
    for r in PARITY_RECORDS:
        terminalreporter.write_line(json.dumps(r))
    out = ROOT / "gpurun_out"
    if out.is_dir():
        (out / "parity_report.json").write_text(json.dumps(PARITY_RECORDS, indent=1))
