"""The stream workspaces' pool (rusty_whisper_amd/csrc/rw_pool.hpp) under
concurrent callers, on the CPU: exclusive hold per stream, no buffer freed or
grown under a holder, every buffer freed once.  Built with g++ under
ThreadSanitizer and AddressSanitizer (tests/native/pool_stress.cpp)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "rusty_whisper_amd", "csrc")


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
@pytest.mark.parametrize("sanitizer", ["thread", "address"])
def test_pool_stress(tmp_path, sanitizer):
    exe = str(tmp_path / f"pool_stress_{sanitizer}")
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", f"-fsanitize={sanitizer}", f"-I{CSRC}",
                    os.path.join(HERE, "native", "pool_stress.cpp"), "-o", exe, "-pthread"], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "bad=0" in r.stdout
    assert "WARNING: ThreadSanitizer" not in r.stderr
