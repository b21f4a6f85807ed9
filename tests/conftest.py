"""Test configuration: import paths and the ``gpu`` marker.

``gfx906-fa-vllm_amd/`` is put on sys.path the way the reference puts its
``extension/`` directory there (its modules are top-level), plus the repo root
(``oracle``) and the offline ``vllm`` stub."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "tests", "vllm_stub"), ROOT, os.path.join(ROOT, "gfx906-fa-vllm_amd"),
          os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
