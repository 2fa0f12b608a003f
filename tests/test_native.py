"""The native tier driver (tests/native/tier_driver.cpp), built by __graft_entry__.build().

CPU: its host-only checks -- the container reader on mutated safetensors headers and
the host segment builder against the oracle, single-threaded and from five threads --
with the library's host side under AddressSanitizer (leak detection on) and
ThreadSanitizer.
GPU: the two-thread store/compute drive of the HBM tier (prefetch, slot reuse, REPIN,
tier tables, the drop-in and device-resident blocks) checked against the oracle, plain
and with the host side under AddressSanitizer."""
import os
import subprocess

import pytest

NATIVE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "native", "_build")
ENV_SAN = {"address": {"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=1"},
           "thread": {"TSAN_OPTIONS": "halt_on_error=1"}}


def run(exe, args, extra_env=None, timeout=300):
    path = os.path.join(NATIVE, exe)
    if not os.path.exists(path):
        pytest.skip(f"{path} not built (run __graft_entry__.build())")
    env = dict(os.environ, **(extra_env or {}))
    p = subprocess.run([path] + args, capture_output=True, text=True, timeout=timeout, env=env)
    print(p.stdout, p.stderr[-4000:], flush=True)
    return p


@pytest.mark.parametrize("san", ["address", "thread"])
def test_host_checks_under_sanitizer(san):
    p = run(f"tier_driver_{san}", ["host", "3000"], ENV_SAN[san])
    assert p.returncode == 0
    assert "0 failures" in p.stdout


@pytest.mark.parametrize("san", ["address", "thread"])
def test_host_entry_points_from_threads(san):
    """Four threads reading containers and building segments while a fifth changes options,
    reads and resets the counters and makes refused calls."""
    p = run(f"tier_driver_{san}", ["host-threads", "300"], ENV_SAN[san])
    assert p.returncode == 0
    assert "host threads: 0 failures" in p.stdout


@pytest.mark.gpu
def test_tier_drive_on_the_device():
    p = run("tier_driver", ["4"])
    assert p.returncode == 0 and "0 failures" in p.stdout


@pytest.mark.gpu
def test_tier_drive_under_asan():
    """The device drive with the library's host side under AddressSanitizer.  (Under
    ThreadSanitizer the ROCm runtime finds no device, so the threaded device drive runs
    under ASan only; the host-only entry points are threaded under TSan above.)"""
    # the HIP runtime keeps allocations until exit and maps device memory itself
    env = {"ASAN_OPTIONS": "detect_leaks=0:protect_shadow_gap=0:abort_on_error=1"}
    p = run("tier_driver_address", ["2"], env)
    assert p.returncode == 0 and "0 failures" in p.stdout
