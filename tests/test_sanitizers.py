"""The block manager's host C++ (csrc/block_manager.cpp, no device code) under
AddressSanitizer and UndefinedBehaviorSanitizer: tests/sanitize/bm_fuzz.cpp
drives random allocate / free / move / complete sequences through the C ABI,
including calls suspended for reclaim, their resumption and cancellation and
frees of the requests they hold, and checks the bookkeeping after every step.
Any memory error, leak or undefined behaviour ends the run with an error."""
import os
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.fixture(scope="module")
def fuzz_binary(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ is not available")
    out = tmp_path_factory.mktemp("bm_fuzz") / "bm_fuzz"
    cmd = [gxx, "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-Wall",
           str(ROOT / "tests" / "sanitize" / "bm_fuzz.cpp"),
           str(ROOT / "aegaeon_amd" / "csrc" / "block_manager.cpp"), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    return out


@pytest.mark.parametrize("seed", [1, 2, 3, 4, 5, 6])
def test_block_manager_under_sanitizers(fuzz_binary, seed):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    res = subprocess.run([str(fuzz_binary), str(seed), "4000"], capture_output=True, text=True,
                         env=env, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "runtime error" not in res.stderr, res.stderr  # UBSan reports
    seen = dict((k, int(v)) for k, v in re.findall(r"(\w+)=(\d+)", res.stdout))
    # the paths the run must have taken
    for path in ("allocate_suspended", "swap_in_suspended", "swap_out_suspended", "resume_ok",
                 "cancel", "free_while_suspended", "swap_in_ok", "swap_out_ok"):
        assert seen.get(path, 0) > 0, (path, res.stdout)
