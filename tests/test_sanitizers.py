"""Host-code sanitizers: libnova_run's parser and planner (plain C++ over
program text) built with AddressSanitizer and UndefinedBehaviorSanitizer,
with any finding fatal, then the CPU planner tests run against that build
in a child process.  No GPU: planning makes no HIP call."""
import os
import subprocess
import sys

import pytest

from conftest import REPO

CLANG = "/opt/rocm/llvm/bin/clang++"


def _asan_runtime():
    try:
        out = subprocess.run([CLANG, "-print-file-name=libclang_rt.asan-x86_64.so"],
                             capture_output=True, text=True, timeout=60).stdout.strip()
    except (OSError, subprocess.TimeoutExpired):
        return None
    return out if out and os.path.isabs(out) and os.path.exists(out) else None


def test_planner_under_asan_and_ubsan(tmp_path):
    if not os.path.exists(CLANG) or _asan_runtime() is None:
        pytest.skip("no clang++ with the AddressSanitizer runtime in this image")
    pkg = os.path.join(REPO, "nova-compiler_amd")
    if not os.path.exists(os.path.join(pkg, "libnova_hip.so")):
        pytest.skip("libnova_hip.so not built")
    lib = str(tmp_path / "libnova_run_asan.so")
    build = [CLANG, "-std=c++17", "-O1", "-g", "-fPIC", "-shared", "-fno-omit-frame-pointer",
             "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
             "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", "-I" + os.path.join(REPO, "include"),
             os.path.join(pkg, "runtime", "nova_run.cpp"), "-o", lib, "-L" + pkg, "-lnova_hip",
             "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath," + pkg, "-Wl,-rpath,/opt/rocm/lib"]
    r = subprocess.run(build, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    script = tmp_path / "run.py"
    script.write_text(
        "import sys\n"
        f"sys.path[:0] = [{pkg!r}, {os.path.join(REPO, 'tests')!r}, {os.path.join(REPO, 'oracle')!r}]\n"
        "import nova_run\n"
        f"nova_run.LIB_PATH = {lib!r}\n"
        "import pytest\n"
        "sys.exit(pytest.main(['-q', '-x', '-m', 'not gpu', '-p', 'no:cacheprovider', "
        f"{os.path.join(REPO, 'tests', 'test_run_plan.py')!r}, "
        f"{os.path.join(REPO, 'tests', 'test_forms.py')!r}]))\n")
    env = dict(os.environ, LD_PRELOAD=_asan_runtime(), ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([sys.executable, str(script)], capture_output=True, text=True, env=env,
                       cwd=str(tmp_path), timeout=900)
    assert r.returncode == 0, (r.stdout[-3000:], r.stderr[-3000:])
    assert "passed" in r.stdout


def test_c_abi_validation_under_asan_and_ubsan(tmp_path):
    """The C ABI's host-side validation (nova_hip_abi.hip: descriptor, shape,
    stride and flag checks) built with ASan and UBSan on the host pass
    only, linked with the other translation units as built, then the C-ABI
    tests (which make no HIP call) against that library."""
    if not os.path.exists(CLANG) or _asan_runtime() is None:
        pytest.skip("no clang++ with the AddressSanitizer runtime in this image")
    pkg = os.path.join(REPO, "nova-compiler_amd")
    build_dir = os.path.join(pkg, "_build")
    objs = [os.path.join(build_dir, f) for f in sorted(os.listdir(build_dir))
            if f.endswith(".o") and f != "nova_hip_abi.o"] if os.path.isdir(build_dir) else []
    if len(objs) < 5:
        pytest.skip("the library's objects are not built (make -C nova-compiler_amd)")
    hipcc = "/opt/rocm/bin/hipcc"
    abi = str(tmp_path / "nova_hip_abi.o")
    host_san = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                "-Xarch_host", "-fno-sanitize-recover=all"]
    r = subprocess.run([hipcc, "--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-fPIC",
                        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"] + host_san +
                       ["-c", os.path.join(pkg, "csrc", "nova_hip_abi.hip"), "-o", abi],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    lib = str(tmp_path / "libnova_hip.so")
    r = subprocess.run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC"] + host_san +
                       [abi] + objs + ["-o", lib], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    script = tmp_path / "run.py"
    script.write_text(
        "import sys\n"
        f"sys.path[:0] = [{pkg!r}, {os.path.join(REPO, 'tests')!r}, {os.path.join(REPO, 'oracle')!r}]\n"
        "import nova_hip\n"
        f"nova_hip.LIB_PATH = {lib!r}\n"
        "import pytest\n"
        "sys.exit(pytest.main(['-q', '-x', '-m', 'not gpu', '-p', 'no:cacheprovider', "
        f"{os.path.join(REPO, 'tests', 'test_abi.py')!r}]))\n")
    env = dict(os.environ, LD_PRELOAD=_asan_runtime(), ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([sys.executable, str(script)], capture_output=True, text=True, env=env,
                       cwd=str(tmp_path), timeout=900)
    assert r.returncode == 0, (r.stdout[-3000:], r.stderr[-3000:])
    assert "passed" in r.stdout
