"""Test configuration: the `gpu` marker (tests that need an MI355X), and import paths for the package under
splash-desktop_amd/ and for the CPU oracle under oracle/ (which only tests and the checkers load)."""
import pathlib
import sys

ROOT = pathlib.Path(__file__).resolve().parent.parent
for path in (ROOT / "splash-desktop_amd", ROOT / "oracle", ROOT / "tests"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X); run with -m gpu")
