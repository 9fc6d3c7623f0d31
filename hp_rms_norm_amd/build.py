"""In-tree build of the native libraries of hp_rms_norm_amd.

    libhprms.so        the gfx950 kernels and their C ABI (hipcc)
    _C.so              the extension module that registers torch.ops.hp_rms_norm.*
                       on top of it (g++)
    libhprms_bench.so  bench and test library, not part of the product: the same
                       C ABI plus the kernel shapes only the tuning sweeps use and
                       the ceiling kernels (hprms_ceiling.hip)

All land next to this file, so they travel with the source tree.  Run
``python hp_rms_norm_amd/build.py [all|product|kernels|torch|oracle|tests]`` (or
``__graft_entry__.build()``; ``product``, the two product libraries, is what
``pip install`` builds) -- as a script, not with ``-m``: importing it through
the package would run the package's __init__, which needs the libraries this
builds.  No GPU is needed: hipcc cross-compiles for gfx950.
"""
import os
import shutil
import subprocess
import sys
import sysconfig
import tempfile

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

KERNEL_LIB = os.path.join(PKG, "libhprms.so")
TORCH_LIB = os.path.join(PKG, "_C.so")
BENCH_LIB = os.path.join(PKG, "libhprms_bench.so")

ARCH = "gfx950"
# Packed fp32 VALU ops stay off: plain fp32 code is what the kernels need, and
# it keeps the generated arithmetic to ordinary IEEE binary32 instructions.
# The leading scalar arguments of every kernel (up to 10 arguments within the
# first 14 dwords of the argument block) are preloaded into SGPRs at wave
# launch (gfx950 kernarg preload): the fused kernels put what their row loop
# needs there.
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-Wall", f"--offload-arch={ARCH}",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-mllvm", "-amdgpu-kernarg-preload-count=10"]


def _report(cmd, p_returncode, text):
    out = "\n".join(line for line in text.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in line)
    if out.strip():
        print(out, flush=True)
    if p_returncode != 0:
        raise RuntimeError(f"build step failed ({p_returncode}): {' '.join(cmd)}")


def _run(cmd):
    print("+", " ".join(cmd), flush=True)
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    _report(cmd, p.returncode, p.stdout)


def _run_parallel(cmds):
    """Runs the commands at once (each compiles one translation unit)."""
    for cmd in cmds:
        print("+", " ".join(cmd), flush=True)
    procs = [subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True) for cmd in cmds]
    outs = [p.communicate()[0] for p in procs]
    for cmd, p, text in zip(cmds, procs, outs):
        _report(cmd, p.returncode, text)


def _atomic(dst, build_fn):
    tmp = dst + ".tmp"
    build_fn(tmp)
    os.replace(tmp, dst)


def build_kernels(bench=True):
    """Compiles every translation unit of csrc/ at once into a scratch
    directory, then links libhprms.so and (with `bench`) libhprms_bench.so.
    The two share the variant and general-tier objects; hprms.hip is compiled
    once per library (HPRMS_BENCH_BUILD adds the bench-only shapes and entry
    point)."""
    hipcc = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
    units = [("hprms.hip", []), ("hprms_unaligned.hip", []), ("hprms_tail.hip", []), ("hprms_general.hip", [])]
    if bench:
        units += [("hprms.hip", ["-DHPRMS_BENCH_BUILD"]), ("hprms_ceiling.hip", [])]
    with tempfile.TemporaryDirectory(prefix="hprms_build_") as tmp:
        objs = [os.path.join(tmp, f"{i}_{name}.o") for i, (name, _) in enumerate(units)]
        _run_parallel([[hipcc, *HIP_FLAGS, *defs, "-c", f"-I{INCLUDE}", f"-I{CSRC}", os.path.join(CSRC, name),
                        "-o", obj] for (name, defs), obj in zip(units, objs)])
        product, shared, bench_objs = objs[0], objs[1:4], objs[4:]
        _atomic(KERNEL_LIB, lambda out: _run([hipcc, *HIP_FLAGS, "-shared", product, *shared, "-o", out]))
        if bench:
            _atomic(BENCH_LIB, lambda out: _run([hipcc, *HIP_FLAGS, "-shared", *bench_objs, *shared, "-o", out]))


def build_torch_binding():
    import torch
    from torch.utils import cpp_extension

    cxx = shutil.which("g++") or "c++"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    incs = [f"-I{p}" for p in cpp_extension.include_paths()] + [
        f"-I{sysconfig.get_paths()['include']}", f"-I{INCLUDE}", f"-I{ROCM}/include"]
    tlib = cpp_extension.library_paths()[0]
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wno-unused-parameter",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           *incs, os.path.join(CSRC, "torch_binding.cpp"),
           f"-L{PKG}", "-lhprms", f"-L{tlib}", "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch",
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{tlib}", "-Wl,--no-as-needed"]
    _atomic(TORCH_LIB, lambda out: _run(cmd + ["-o", out]))


def build_oracle():
    oracle_dir = os.path.join(ROOT, "oracle")
    if os.path.exists(os.path.join(oracle_dir, "Makefile")):
        _run(["make", "-s", "-B", "-C", oracle_dir])


def build_test_programs():
    """tests/c_gpu_caller (gcc): the C ABI driven from a plain C program on
    the GPU, checked against the oracle; test infrastructure."""
    tests_dir = os.path.join(ROOT, "tests")
    if os.path.exists(os.path.join(tests_dir, "Makefile")) and shutil.which("gcc"):
        _run(["make", "-s", "-B", "-C", tests_dir])


def build_all():
    build_kernels()
    build_torch_binding()
    build_oracle()
    build_test_programs()


def build_product():
    """libhprms.so and _C.so only: what an installed package holds."""
    build_kernels(bench=False)
    build_torch_binding()


if __name__ == "__main__":
    what = sys.argv[1:] or ["all"]
    for w in what:
        {"all": build_all, "product": build_product, "kernels": build_kernels, "torch": build_torch_binding,
         "oracle": build_oracle, "tests": build_test_programs}[w]()
