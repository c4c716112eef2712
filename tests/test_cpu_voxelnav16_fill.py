"""VoxelNav16's grid fill on the host: the packed cells a reset writes against
the cells read field by field from the same draws
(tests/native/voxelnav16_fill.cpp)."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_voxelnav16_fill_host(tmp_path):
    exe = str(tmp_path / "voxelnav16_fill")
    subprocess.run(["g++", "-std=c++17", "-O2", "-Wall", "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "native", "voxelnav16_fill.cpp"), "-o", exe], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "0 failures" in r.stdout, r.stdout + r.stderr
