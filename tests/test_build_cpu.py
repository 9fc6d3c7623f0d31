"""The build from a clean tree, on the CPU: a copy of the sources without any
built library goes through __graft_entry__.build() (hipcc for gfx950, g++ for
the torch binding, gcc for the oracle) and the package then imports.  The
libraries are git-ignored, so this is the state a fresh checkout starts in."""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc not found")
def test_build_from_a_clean_tree(tmp_path):
    skip = shutil.ignore_patterns("*.so", "*.so.tmp*", "__pycache__", "*.o")
    for d in ("hp_rms_norm_amd", "hp_rms_norm", "include", "oracle"):
        shutil.copytree(os.path.join(ROOT, d), tmp_path / d, ignore=skip)
    shutil.copy(os.path.join(ROOT, "__graft_entry__.py"), tmp_path)
    assert not list(tmp_path.rglob("*.so"))
    p = subprocess.run([sys.executable, "-c", "import __graft_entry__ as g; g.build()"], cwd=tmp_path,
                       capture_output=True, text=True, timeout=1200)
    assert p.returncode == 0, p.stdout[-3000:] + p.stderr[-3000:]
    assert "build: ok" in p.stdout
    for lib in ("hp_rms_norm_amd/libhprms.so", "hp_rms_norm_amd/_C.so", "hp_rms_norm_amd/libhprms_bench.so",
                "oracle/libhprms_oracle.so"):
        assert (tmp_path / lib).exists(), lib
