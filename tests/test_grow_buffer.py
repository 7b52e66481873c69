"""The grow-only workspace rules of the entry points that allocate (the float-code row-band
and stream paths, the fp32 filter gradient), tested on the CPU: tests/cpp/grow_buffer_test.cpp
is built with g++ against my_own_cnn_amd/csrc/grow_buffer.h (host code only) and run."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_grow_buffer_rules(tmp_path):
    exe = tmp_path / "grow_buffer_test"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", f"-I{ROOT / 'my_own_cnn_amd' / 'csrc'}",
                    str(ROOT / "tests" / "cpp" / "grow_buffer_test.cpp"), "-o", str(exe)], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.strip() == "ok"
