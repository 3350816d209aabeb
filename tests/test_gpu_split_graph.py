"""The drop-in attn_decode_split (engine.cu:396-464) allocates nothing and
is capturable: split + combine captured into a HIP graph as a fresh
process's first split call, on a fresh stream, then replayed bit-identical
to eager calls (partials included), in a child process so that no earlier
test has called the entry (tests/split_capture_child.py)."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def test_split_first_call_under_capture(cia, dev):
    r = subprocess.run([sys.executable, "-u", os.path.join(HERE, "split_capture_child.py")],
                       capture_output=True, text=True, timeout=300)
    print(r.stdout[-4000:])
    print(r.stderr[-4000:])
    assert r.returncode == 0, f"child exited {r.returncode}: {r.stderr[-2000:]}"
    assert "split capture ok" in r.stdout
