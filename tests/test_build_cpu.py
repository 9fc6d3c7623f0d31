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


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc not found")
def test_wheel_holds_the_product_and_imports_outside_the_tree(tmp_path):
    """setup.py (the reference's install path: the distribution hp_rms_norm)
    builds a wheel from a clean copy of the sources without network or build
    isolation; the wheel holds both packages and the two product libraries,
    not the bench library, and the packages import from the unpacked wheel
    in a process started outside the source tree."""
    import zipfile
    src = tmp_path / "src"
    skip = shutil.ignore_patterns("*.so", "*.so.tmp*", "__pycache__", "*.o")
    for d in ("hp_rms_norm_amd", "hp_rms_norm", "include"):
        shutil.copytree(os.path.join(ROOT, d), src / d, ignore=skip)
    shutil.copy(os.path.join(ROOT, "setup.py"), src)
    p = subprocess.run([sys.executable, "-m", "pip", "wheel", "--no-build-isolation", "--no-deps", "--no-index",
                        "-w", str(tmp_path / "whl"), str(src)], capture_output=True, text=True, timeout=1200)
    assert p.returncode == 0, p.stdout[-3000:] + p.stderr[-3000:]
    (whl,) = (tmp_path / "whl").glob("hp_rms_norm-*.whl")
    assert "linux_x86_64" in whl.name
    names = zipfile.ZipFile(whl).namelist()
    base = {n.split("/purelib/", 1)[-1] for n in names if "/purelib/" in n}
    assert {"hp_rms_norm/__init__.py", "hp_rms_norm/ops.py", "hp_rms_norm_amd/__init__.py",
            "hp_rms_norm_amd/ops.py", "hp_rms_norm_amd/abi.py", "hp_rms_norm_amd/libhprms.so",
            "hp_rms_norm_amd/_C.so"} <= base
    assert not any("bench" in n or "oracle" in n for n in names)
    zipfile.ZipFile(whl).extractall(tmp_path / "site")
    (purelib,) = (tmp_path / "site").glob("*.data/purelib")
    code = ("import hp_rms_norm, hp_rms_norm_amd, torch; from hp_rms_norm import _C; "
            "print(hp_rms_norm_amd.__file__); print(_C.__file__); print(torch.ops.hp_rms_norm.rms_norm)")
    env = dict(os.environ, PYTHONPATH=str(purelib))
    p = subprocess.run([sys.executable, "-c", code], cwd=tmp_path, env=env, capture_output=True, text=True,
                       timeout=300)
    assert p.returncode == 0, p.stderr[-3000:]
    lines = p.stdout.split()
    assert lines[0].startswith(str(purelib)) and lines[1].startswith(str(purelib)), p.stdout
