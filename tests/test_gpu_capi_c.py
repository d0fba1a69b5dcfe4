"""The C ABI from a plain C program (thintnpu_amd/capi_selftest, built by
thintnpu_amd/build.py): hipMalloc'd buffers, its own stream and no PyTorch in
the process.  It checks exact results on the host and exits 0 when all pass."""
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

SELFTEST = Path(__file__).resolve().parent.parent / "thintnpu_amd" / "capi_selftest"


def test_plain_c_consumer(gpu):
    assert SELFTEST.exists(), f"{SELFTEST} is not built; run __graft_entry__.build()"
    proc = subprocess.run([str(SELFTEST)], capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "capi selftest ok" in proc.stdout
