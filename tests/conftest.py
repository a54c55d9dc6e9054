import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path)")
    config.addinivalue_line("markers", "slow: long CPU-side reference runs")


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """Per test, the worst parity margin its comparisons reached: max abs
    error, and err / (atol + rtol*|ref|) (the test fails above 1.0)."""
    from tests.tol import MARGINS
    if not MARGINS:
        return
    worst = {}
    for node, what, mx, rel, ratio in MARGINS:
        w = worst.get(node)
        if w is None:
            worst[node] = [mx, ratio, what, 1]
        else:
            w[3] += 1
            if mx > w[0]:
                w[0] = mx
            if ratio > w[1]:
                w[1], w[2] = ratio, what
    tr = terminalreporter
    tr.write_sep("-", "parity margins (max |err|; worst err/bound, 1.0 = tolerance)")
    for node, (mx, ratio, what, n) in worst.items():
        tr.write_line(f"{mx:9.3g}  {ratio:6.3f}  n={n:<3d} {node}  [{what}]")
    tr.write_line(f"overall: max err/bound {max(w[1] for w in worst.values()):.3f} over "
                  f"{len(MARGINS)} comparisons in {len(worst)} tests")
