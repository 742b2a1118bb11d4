"""Host unit test of the stream-K arrival protocol: the counter logic of
spinn_amd/csrc/sk_arrive.h (what the conv kernel runs over system-scope HIP
atomics) compiled with g++ over std::atomic, on garbage, stale, replayed,
raced, hostile and concurrent counters; a broken protocol must report -1
(the kernel then sets the host-visible status word) instead of leaving a
tile silently unwritten."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def test_streamk_arrival_protocol(tmp_path):
    gxx = shutil.which("g++")
    if not gxx:
        pytest.skip("g++ not available")
    exe = tmp_path / "arrive_test"
    subprocess.run([gxx, "-std=c++17", "-O1", "-pthread", "-I", str(ROOT / "spinn_amd" / "csrc"),
                    str(ROOT / "tests" / "streamk_arrive" / "arrive_test.cc"), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.count("ok  ") == 9
