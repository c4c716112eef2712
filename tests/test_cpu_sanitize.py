"""The CPU oracle (the checker every parity test trusts) under
AddressSanitizer + UndefinedBehaviorSanitizer and under ThreadSanitizer:
tests/sanitize/drive.cpp calls every oracle entry point for every env, both
precisions and several thread counts (the oracle shards envs and rows over
std::thread). Any sanitizer report fails the run."""
import os
import subprocess

import pytest

SAN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "sanitize")


@pytest.fixture(scope="module")
def drivers():
    subprocess.run(["make", "-s", "-j2", "-C", SAN], check=True)
    return os.path.join(SAN, "build")


@pytest.mark.parametrize("which", ["asan", "tsan"])
def test_oracle_under_sanitizer(drivers, which):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1", UBSAN_OPTIONS="print_stacktrace=1",
               TSAN_OPTIONS="halt_on_error=1")
    r = subprocess.run([os.path.join(drivers, f"drive_{which}")], env=env, capture_output=True, text=True,
                       timeout=600)
    if which == "tsan" and r.returncode != 0 and "unexpected memory mapping" in r.stderr:
        pytest.skip("ThreadSanitizer cannot map its shadow memory on this kernel")
    assert r.returncode == 0, r.stderr[-4000:]
    assert "0 failures" in r.stdout
