"""Host-side AddressSanitizer + UndefinedBehaviorSanitizer run over the C ABI.

``tests/host_sanitizer/build_and_run.sh`` builds libnqamd with both sanitizers
on its host code and runs ``abi_checks.cpp``: argument errors of the entry
points, and the launch planning of decode and prefill calls (descriptor checks,
geometry, tile and wave choice, kernel-argument packing) over the Qwen3-8B
shapes at 1-300 tokens, which ends in NQ_ERR_LAUNCH where no GPU is visible.
Any sanitizer report aborts the driver. CPU only: where a GPU is visible the
driver runs nothing (exit 77) and the test is skipped.
"""

import shutil
import subprocess
from pathlib import Path

import pytest

SCRIPT = Path(__file__).resolve().parent / "host_sanitizer" / "build_and_run.sh"


def test_c_abi_host_code_under_asan_and_ubsan(tmp_path):
    if not SCRIPT.exists() or shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists():
        pytest.skip("the sanitizer recipe or hipcc is not available")
    result = subprocess.run(["bash", str(SCRIPT), str(tmp_path / "san")], capture_output=True, text=True,
                            timeout=900)
    if result.returncode == 77:
        pytest.skip("a GPU is visible: the host-only driver ran nothing")
    tail = "\n".join((result.stdout + result.stderr).splitlines()[-30:])
    assert result.returncode == 0, tail
    assert "ok: 0 failed checks" in result.stdout, tail
