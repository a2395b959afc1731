"""AddressSanitizer + UndefinedBehaviorSanitizer runs of the CPU-side code
(CPU only; each run is a subprocess, because a sanitizer runtime must be
preloaded into the interpreter):

* the CPU restatement (oracle/), built by `make -C oracle asan`, under the
  oracle test files;
* the C ABI's host code (brush_amd/csrc/api.hip: argument checks, context
  creation without a device), its host half built with -Xarch_host
  sanitizers and linked with the other objects of the regular build, under
  the C-ABI tests.

Each environment is first shown to catch a planted heap overflow in a
throwaway C function, so a clean run means the sanitizer was active."""
import glob
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "brush_amd", "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ASAN_OPTIONS = "detect_leaks=0:abort_on_error=1:halt_on_error=1"


def _gcc_runtimes():
    libs = []
    for name in ("libasan.so", "libubsan.so"):
        path = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
        if not os.path.isabs(path) or not os.path.exists(path):
            pytest.skip(f"gcc has no {name}")
        libs.append(path)
    return ":".join(libs)


def _clang_asan_runtime():
    found = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not found or not os.path.exists(HIPCC):
        pytest.skip("no clang AddressSanitizer runtime")
    return found[-1]


def _run(args, env_extra, timeout=600):
    env = dict(os.environ, ASAN_OPTIONS=ASAN_OPTIONS, UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
               OMP_NUM_THREADS="4", **env_extra)
    return subprocess.run(args, cwd=ROOT, env=env, capture_output=True, text=True, timeout=timeout)


def _canary(tmp_path, cc, flags, preload):
    """A heap overflow in a throwaway library, called through ctypes in the
    same environment: the sanitizer must report it."""
    src = tmp_path / "canary.c"
    src.write_text("#include <stdlib.h>\nint canary(int i) { int* p = malloc(4 * sizeof(int)); "
                   "int v = p[i]; free(p); return v; }\n")
    lib = tmp_path / "libcanary.so"
    res = subprocess.run([*cc, *flags, "-shared", "-fPIC", "-o", str(lib), str(src)], capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    code = f"import ctypes; ctypes.CDLL({str(lib)!r}).canary(4)"
    res = _run([sys.executable, "-c", code], {"LD_PRELOAD": preload}, timeout=120)
    assert res.returncode != 0 and "AddressSanitizer" in res.stderr, res.stderr[-2000:]


def test_oracle_under_asan_and_ubsan(tmp_path):
    preload = _gcc_runtimes()
    res = subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "asan"], capture_output=True, text=True)
    assert res.returncode == 0, res.stdout + res.stderr
    _canary(tmp_path, ["gcc"], ["-fsanitize=address,undefined", "-g"], preload)
    tests = [os.path.join("tests", f) for f in ("test_oracle.py", "test_oracle_backward.py",
                                                 "test_oracle_camera.py", "test_oracle_train.py")]
    res = _run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", *tests],
               {"LD_PRELOAD": preload, "BH_ORACLE_LIB": os.path.join(ROOT, "oracle", "liboracle_asan.so")})
    assert res.returncode == 0, (res.stdout[-3000:] + res.stderr[-3000:])
    assert "runtime error" not in res.stderr and "AddressSanitizer" not in res.stderr, res.stderr[-3000:]


def test_c_abi_host_code_under_asan_and_ubsan(tmp_path):
    preload = _clang_asan_runtime()
    objs = sorted(glob.glob(os.path.join(BUILD, "*.o")))
    if not any(o.endswith("api.o") for o in objs):
        pytest.skip("the library has not been built (__graft_entry__.build())")
    _canary(tmp_path, ["/opt/rocm/llvm/bin/clang"], ["-fsanitize=address,undefined", "-shared-libsan", "-g"],
            preload)
    san = []
    for flag in ("-fsanitize=address", "-fsanitize=undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"):
        san += ["-Xarch_host", flag]
    api_o = str(tmp_path / "api.o")
    from brush_amd import build as B

    flags = [f for f in B.FLAGS if f not in ("-shared", "-Rpass-analysis=kernel-resource-usage")]
    res = subprocess.run([HIPCC, *flags, "-g", *san, "-c", "-o", api_o, os.path.join(ROOT, "brush_amd", "csrc",
                                                                                       "api.hip")],
                         capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-3000:]
    lib = str(tmp_path / "libbrush_hip_asan.so")
    others = [o for o in objs if not o.endswith("api.o")]
    res = subprocess.run([HIPCC, "--offload-arch=gfx950", "-fPIC", "-shared", "-Xarch_host", "-fsanitize=address",
                          "-Xarch_host", "-fsanitize=undefined", "-Xarch_host", "-shared-libsan", "-o", lib, api_o,
                          *others, *B.LINK_LIBS], capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-3000:]
    res = _run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", "-m", "not gpu",
                os.path.join("tests", "test_cabi.py")], {"LD_PRELOAD": preload, "BH_LIB_PATH": lib})
    assert res.returncode == 0, (res.stdout[-3000:] + res.stderr[-3000:])
    assert "passed" in res.stdout and "AddressSanitizer" not in res.stderr, res.stdout[-2000:]
