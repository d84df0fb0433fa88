"""pytest configuration: the ``gpu`` marker and import paths.

Tests marked ``gpu`` need an MI355X (they call libphantom_moe.so); the rest
run on the CPU (oracle, host logic, library symbol table)."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "solution-is-all-you-need_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU (MI355X); runs the HIP library")
