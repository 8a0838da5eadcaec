"""Host-side sanitizers over the C ABI (CPU only, with no GPU visible).

The library is rebuilt with AddressSanitizer and UndefinedBehaviorSanitizer on
its host half (each flag behind hipcc's -Xarch_host; the gfx950 code is built
as usual) into a temporary directory.  Two child processes then run with the
ASan runtime preloaded and that build named by DELS_LIBRARY_PATH:
  * the C-ABI host tests (test_capi_host.py): exports, workspace sizes and the
    argument checks with their messages;
  * abi_fuzz.py: every entry point called with random, mostly invalid
    arguments (NULL and misaligned pointers, negative and huge extents,
    NaN/inf scalars, workspaces too small).
Every sanitizer finding aborts the child, which fails the test.  Device
pointers in these calls are fake, so the test refuses to run where a GPU is
visible.
"""

import importlib.util
import os
import shutil
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SAN = "address,undefined"
HOST_FLAGS = ("-Xarch_host", "-fsanitize=" + SAN, "-Xarch_host", "-fno-sanitize=vptr",
              "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer",
              "-Xarch_host", "-g")
LINK_FLAGS = ("-Xarch_host", "-fsanitize=" + SAN)


def _asan_runtime():
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    clang = os.path.join(rocm, "llvm", "bin", "clang")
    if not os.path.exists(clang):
        return None
    out = subprocess.run([clang, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    path = out.stdout.strip()
    return path if out.returncode == 0 and os.path.isabs(path) and os.path.exists(path) else None


def _gpu_visible():
    import torch

    return torch.cuda.device_count() > 0


@pytest.fixture(scope="module")
def sanitized_lib(tmp_path_factory):
    if _gpu_visible():
        pytest.skip("fake device pointers are passed: runs only where no GPU is visible")
    spec = importlib.util.spec_from_file_location("dels_build", os.path.join(REPO, "dels-spec_amd", "build.py"))
    build = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(build)
    runtime = _asan_runtime()
    if runtime is None or shutil.which(build.hipcc()) is None:
        pytest.skip("hipcc or the clang ASan runtime is not available")
    lib = str(tmp_path_factory.mktemp("san") / "libdels_mi355x_san.so")
    build.build(lib_path=lib, extra_flags=HOST_FLAGS, link_flags=LINK_FLAGS)
    return lib, runtime


def _run(sanitized_lib, argv, timeout):
    lib, runtime = sanitized_lib
    env = dict(os.environ)
    env.update(DELS_LIBRARY_PATH=lib, LD_PRELOAD=runtime, HIP_VISIBLE_DEVICES="-1",
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:exitcode=86",
               UBSAN_OPTIONS="print_stacktrace=1:exitcode=86")
    p = subprocess.run([sys.executable, *argv], cwd=REPO, env=env, capture_output=True, text=True, timeout=timeout)
    text = p.stdout + p.stderr
    assert "Sanitizer" not in text and "runtime error" not in text, text[-4000:]
    assert p.returncode == 0, text[-4000:]
    return text


def test_capi_host_tests_under_sanitizers(sanitized_lib):
    out = _run(sanitized_lib, ["-m", "pytest", "-q", "-p", "no:cacheprovider", "-m", "not gpu",
                               os.path.join("tests", "test_capi_host.py")], timeout=600)
    assert " passed" in out


def test_abi_fuzz_under_sanitizers(sanitized_lib):
    out = _run(sanitized_lib, [os.path.join("tests", "abi_fuzz.py"), "400", "7"], timeout=600)
    assert "no finding" in out
