"""pytest configuration: the `gpu` marker and import paths.

CPU tests (-m "not gpu") exercise the C oracle against closed forms, golden
fixtures and independent numpy restatements, plus the C-ABI library's exported
symbols.  GPU tests (-m gpu) run the HIP path through the C-ABI on cuda:0 and
compare it with the oracle.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path on cuda:0)")
