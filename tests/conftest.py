import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libnuq.so on cuda:0)")


def pytest_terminal_summary(terminalreporter):
    try:
        from tests.gpu_util import WORST
    except Exception:
        return
    if not WORST:
        return
    terminalreporter.write_line("worst observed |gpu - oracle| / sum|w*x| per check (bound factor k):")
    for (family, _), (ratio, k, label) in sorted(WORST.items()):
        terminalreporter.write_line(f"  {family:12s} {ratio:.3e}  (k = {k:.0e})  worst: {label}")
