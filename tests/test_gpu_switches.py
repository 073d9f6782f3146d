"""The library's environment switches, each in its non-default setting
(tests/switch_child.py in a child process, since the library reads them once
per process): EM_STRIP_COPY=0 keeps no strip copies, EM_DECODE_MFMA=0 keeps
2 - 8 registered rows on the row-major kernels. Both leave every product
within the oracle's bound and bit-identical to the path they fall back to.
(The forward pass's switches, read at model creation, are tested in
test_gpu_model.py.)"""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.parametrize("mode,var", [("strip_copy_off", "EM_STRIP_COPY"),
                                      ("decode_mfma_off", "EM_DECODE_MFMA")])
def test_switch_off(mode, var):
    env = dict(os.environ)
    env[var] = "0"
    r = subprocess.run([sys.executable, os.path.join(ROOT, "tests", "switch_child.py"), mode],
                       env=env, capture_output=True, text=True, timeout=240)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout + r.stderr
