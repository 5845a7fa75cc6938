import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


def pytest_terminal_summary(terminalreporter):
    """Error figures of the layer outputs checked in this run (labelled ones):
    the per-token-norm error the tests assert and the element-wise relative
    error over outputs >= 1% of their token's largest."""
    try:
        from moe_cases import LAYER_ERRORS
    except Exception:
        return
    rows = [r for r in LAYER_ERRORS if r[0]]
    if not rows:
        return
    terminalreporter.write_sep("-", "layer output error vs the oracle (bar: per-token norm <= 1e-3)")
    for label, tok, elem, n in rows:
        terminalreporter.write_line(f"{label:40s} per-token {tok:.2e}  element-wise {elem:.2e}  ({n} elements)")
