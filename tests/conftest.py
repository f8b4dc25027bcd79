import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover - torch is part of the image
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


# Parity margins in the run's own summary: every test reports its errors as
# "[parity] <label>: key=value ..." lines on stdout (captured under -q), and
# the terminal summary lists the largest value of each key over the run with
# the case that produced it, so a quiet run shows how close it came to a bar.
_PARITY = {}
_PARITY_COUNT = [0]


def _parse_parity(text, nodeid):
    import re
    for line in text.splitlines():
        i = line.find("[parity] ")
        if i < 0:
            continue
        label, _, rest = line[i + 9:].partition(": ")
        _PARITY_COUNT[0] += 1
        for key, val in re.findall(r"([\w./]+)=([-+0-9.eE]+)", rest):
            try:
                x = float(val)
            except ValueError:
                continue
            if x > _PARITY.get(key, (-1.0, ""))[0]:
                _PARITY[key] = (x, f"{label} ({nodeid.split('::')[-1]})")


def pytest_runtest_logreport(report):
    if report.when == "call" and report.capstdout:
        _parse_parity(report.capstdout, report.nodeid)


def pytest_terminal_summary(terminalreporter):
    if not _PARITY:
        return
    tr = terminalreporter
    tr.section("parity margins")
    tr.write_line(f"{_PARITY_COUNT[0]} parity reports; the largest value of each key "
                  "(bars: outputs 1e-2, gradients 2e-2 of the oracle's max-abs unless the "
                  "test states its own):")
    for key in sorted(_PARITY):
        x, where = _PARITY[key]
        tr.write_line(f"  {key:>22s} = {x:.3e}   {where[:150]}")
