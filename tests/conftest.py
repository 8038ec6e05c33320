"""Test configuration: the ``gpu`` marker and import paths.

``-m "not gpu"`` runs on any host (oracle, golden fixtures, ROM generator, the
C ABI's exports); ``-m gpu`` needs an MI355X and the built native libraries.
"""

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU (MI355X) and the built HIP library")
