"""Host-side AddressSanitizer / UndefinedBehaviorSanitizer build of the C-ABI
library, run on the CPU (no GPU is touched).

Every library source is compiled again with the sanitizers on its host code
only (``-Xarch_host`` before each ``-fsanitize=``; the device code is built
as usual), linked with ``tests/sanitize/capi_check.cpp`` into one
executable, and run.  The driver sweeps every entry point's integer
arguments over extreme values and its tensor pointers over NULL (see the
driver's header); any sanitizer report aborts it.  The build takes about a
minute of CPU time, so the test is marked ``slow``.
"""
import concurrent.futures
import os
import shutil
import subprocess
import tempfile

import pytest

from tests.conftest import ROOT, gpu_available

pytestmark = pytest.mark.slow

SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
       "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer", "-g"]


def test_capi_host_code_under_asan_ubsan():
    from dsa_triton_ascend_amd import build_lib as bl
    try:
        hipcc = bl.hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    if gpu_available():
        pytest.skip("the sweep calls entry points with dummy pointers; it only runs without a GPU")
    work = tempfile.mkdtemp(prefix="dsa_san_")
    try:
        def compile_one(src):
            obj = os.path.join(work, os.path.splitext(os.path.basename(src))[0] + ".o")
            lang = ["-x", "hip"] if src.endswith(".cpp") else []
            cmd = ([hipcc] + lang + bl.common_flags() + bl.PER_SOURCE_FLAGS.get(src, []) + SAN
                   + ["-c", os.path.join(bl.CSRC, src), "-o", obj])
            r = subprocess.run(cmd, capture_output=True, text=True)
            return src, obj, r.returncode, r.stdout + r.stderr

        with concurrent.futures.ThreadPoolExecutor(max_workers=min(6, os.cpu_count() or 1)) as ex:
            results = list(ex.map(compile_one, bl.SOURCES))
        for src, _, rc, log in results:
            assert rc == 0, f"sanitized build of {src} failed:\n{log[-3000:]}"
        exe = os.path.join(work, "capi_check")
        driver = os.path.join(ROOT, "tests", "sanitize", "capi_check.cpp")
        drv_obj = os.path.join(work, "capi_check_main.o")
        cmd = ([hipcc, "-x", "hip", f"--offload-arch={bl.ARCH}", "-std=c++17", "-I", os.path.join(ROOT, "include")]
               + SAN + ["-c", driver, "-o", drv_obj])
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, f"driver build failed:\n{(r.stdout + r.stderr)[-3000:]}"
        cmd = ([hipcc, f"--offload-arch={bl.ARCH}"] + SAN + [drv_obj] + [obj for _, obj, _, _ in results]
               + ["-o", exe, "-lpthread"])
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, f"link failed:\n{(r.stdout + r.stderr)[-3000:]}"
        env = dict(os.environ)
        # the HIP runtime keeps its allocations until exit: leaks are not checked
        env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=0:halt_on_error=1"
        env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
        r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=600)
        out = r.stdout + r.stderr
        assert r.returncode == 0, f"sanitized C-ABI sweep failed (rc {r.returncode}):\n{out[-5000:]}"
        assert "OK" in r.stdout or "SKIP" in r.stdout, out[-2000:]
        print(r.stdout.strip())
    finally:
        shutil.rmtree(work, ignore_errors=True)
