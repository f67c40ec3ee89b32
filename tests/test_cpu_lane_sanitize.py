"""The CPU lane's host code (exact and fast modes, the persistent worker pool, the reused buffers) under the address,
undefined-behaviour and thread sanitizers: tests/native/lane_sanitize.cpp drives it over every trellis format, several
shapes and worker counts, built with g++ together with csrc/cpu_lane.cpp. No GPU."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
SRC = [os.path.join(HERE, "native", "lane_sanitize.cpp"), os.path.join(REPO, "big-moe-small-box_amd", "csrc", "cpu_lane.cpp")]


@pytest.mark.parametrize("san,args", [("address,undefined", []), ("thread", ["small"])])
def test_cpu_lane_under_sanitizer(tmp_path, san, args):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not found")
    exe = str(tmp_path / "lane_sanitize")
    cmd = [gxx, "-std=c++17", "-O1", "-g", f"-fsanitize={san}", "-fno-omit-frame-pointer", "-ffp-contract=off",
           "-Wno-psabi", "-I", os.path.join(REPO, "include"), "-o", exe] + SRC + ["-lpthread"]
    b = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert b.returncode == 0, b.stderr[-4000:]
    env = dict(os.environ, UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", ASAN_OPTIONS="detect_leaks=1",
               TSAN_OPTIONS="halt_on_error=1")
    r = subprocess.run([exe] + args, capture_output=True, text=True, timeout=600, env=env)
    out = r.stdout + r.stderr
    assert r.returncode == 0 and "lane sanitize: 0 mismatches" in out, out[-4000:]
    assert "runtime error" not in out and "Sanitizer" not in out, out[-4000:]
