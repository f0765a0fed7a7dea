"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer, on the
CPU (no GPU is touched).

- The HIP library's host side (archive reader and exporter, config loader,
  and the argument checks of every C-ABI entry point) is built by
  ``make sanitize`` in the package.  It is run through tests/test_abi.py,
  tests/test_archive.py and tests/test_archive_fuzz.py, in a child process
  with clang's ASan runtime preloaded.  tests/cpp/test_archive is linked
  against it and run with leak checks on.
- The CPU oracle (oracle/linear_oracle.c, oracle/model_oracle.c) is built
  by ``make sanitize`` in oracle/, with gcc's runtimes.  It is run through
  the oracle's own test files the same way.

Each child stops at the first report (halt_on_error), and its output is
echoed here.  A positive control makes one out-of-bounds read through each
build and expects the report, so an uninstrumented build cannot pass."""
import glob
import os
import subprocess
import sys
import textwrap

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "qwen2.5-jetson-inference_amd")
HIP_SAN = os.path.join(PKG, "_build_san", "libinfer_linear.so")
ORACLE_SAN = os.path.join(ROOT, "oracle", "_san", "liblinear_oracle.so")
REPORTS = ("ERROR: AddressSanitizer", "ERROR: LeakSanitizer", "runtime error:")


def _clang_asan():
    found = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not found:
        pytest.skip("clang's AddressSanitizer runtime is not installed")
    return found[-1]


def _gcc_asan():
    path = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True,
                          text=True).stdout.strip()
    if not os.path.isabs(path) or not os.path.exists(path):
        pytest.skip("gcc's AddressSanitizer runtime is not installed")
    return path


def _make(directory, target):
    subprocess.run(["make", "-j8", "-C", directory, target], check=True,
                   stdout=subprocess.DEVNULL, stderr=subprocess.PIPE)


def _env(runtime, **extra):
    env = dict(os.environ)
    env.update(LD_PRELOAD=runtime,
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:detect_odr_violation=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", **extra)
    return env


def _run(cmd, env, timeout=900):
    done = subprocess.run(cmd, env=env, cwd=ROOT, capture_output=True, text=True,
                          timeout=timeout)
    return done.returncode, done.stdout + done.stderr


def _pytest(files, env):
    rc, out = _run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider",
                    *files], env)
    print(out[-4000:])
    assert rc == 0 and not any(r in out for r in REPORTS), out[-4000:]


@pytest.fixture(scope="module")
def hip_san():
    _make(PKG, "sanitize")
    return _env(_clang_asan(), INFER_HIP_LIBRARY=HIP_SAN)


@pytest.fixture(scope="module")
def oracle_san():
    _make(os.path.join(ROOT, "oracle"), "sanitize")
    return _env(_gcc_asan(), INFER_ORACLE_LIBRARY=ORACLE_SAN)


def test_library_host_code_is_clean(hip_san):
    _pytest(["tests/test_abi.py", "tests/test_archive.py", "tests/test_archive_fuzz.py"],
            hip_san)


def test_cpp_archive_boundary_is_clean_and_leak_free(hip_san):
    _make(os.path.join(ROOT, "tests", "cpp"), "test_archive_san")
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    rc, out = _run([os.path.join(ROOT, "tests", "cpp", "test_archive_san")], env)
    assert rc == 0 and "PASSED" in out and not any(r in out for r in REPORTS), out[-4000:]


def test_oracle_is_clean(oracle_san):
    _pytest(["tests/test_oracle.py", "tests/test_golden.py", "tests/test_model_oracle.py"],
            oracle_san)


# An export whose tensor claims 4096 + 64 floats over a 4096-float buffer:
# the library reads past the allocation.
_HIP_CONTROL = textwrap.dedent("""
    import ctypes, os, sys, tempfile
    sys.path.insert(0, {pkg!r})
    import numpy as np
    import archive_hip
    lib = archive_hip.load()
    data = np.ones(4096, np.float32)
    shape = (ctypes.c_int64 * 1)(4096 + 64)
    t = archive_hip._ExportTensor(b"model.norm.weight", 1, shape,
                                  data.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    with tempfile.TemporaryDirectory() as d:
        lib.infer_hip_archive_export(os.path.join(d, "x.qbin").encode(), b"w16a16", 64,
                                     ctypes.byref(t), 1, b"", None)
    print("no report")
""")

# A BF16 conversion of 4096 + 64 values out of a 4096-float buffer.
_ORACLE_CONTROL = textwrap.dedent("""
    import sys
    sys.path.insert(0, {oracle!r})
    import numpy as np
    import oracle
    lib = oracle._load()
    src = np.ones(4096, np.float32)
    dst = np.zeros(4096 + 64, np.uint16)
    lib.orc_f32_to_bf16_array(src.ctypes.data, dst.ctypes.data, 4096 + 64)
    print("no report")
""")


def test_positive_control_hip_build_reports_overflow(hip_san):
    rc, out = _run([sys.executable, "-c", _HIP_CONTROL.format(pkg=PKG)], hip_san, timeout=300)
    assert rc != 0 and "AddressSanitizer: heap-buffer-overflow" in out, out[-3000:]
    assert "infer_hip_archive_export" in out, out[-3000:]


def test_positive_control_oracle_build_reports_overflow(oracle_san):
    rc, out = _run([sys.executable, "-c", _ORACLE_CONTROL.format(
        oracle=os.path.join(ROOT, "oracle"))], oracle_san, timeout=300)
    assert rc != 0 and "AddressSanitizer: heap-buffer-overflow" in out, out[-3000:]
    assert "orc_f32_to_bf16_array" in out, out[-3000:]
