"""Memory and undefined-behaviour checks of the CPU-side code (no GPU):
the oracle's C restatement and the host side of the C ABI (argument
validation, dispatch up to the device check, per-thread error reporting),
each built with AddressSanitizer and UBSan and driven through edge cases by
the drivers in tests/sanitize/.  The HIP host code is built with the
sanitizers on the host pass only (-Xarch_host)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = os.path.join(ROOT, "tests", "sanitize")
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
           UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")


def run(cmd, **kw):
    r = subprocess.run(cmd, capture_output=True, text=True, **kw)
    assert r.returncode == 0, f"{' '.join(cmd)}\n{r.stdout}\n{r.stderr}"
    return r


def test_oracle_under_asan_ubsan(tmp_path):
    if not shutil.which("gcc"):
        pytest.skip("gcc not found")
    exe = str(tmp_path / "oracle_san")
    run(["gcc", "-O1", "-g", "-std=c11", "-D_POSIX_C_SOURCE=200809L", "-fno-omit-frame-pointer",
         "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
         os.path.join(SAN, "oracle_driver.c"), os.path.join(ROOT, "oracle", "ortho_oracle.c"),
         os.path.join(ROOT, "oracle", "cpu_baseline.c"), "-o", exe, "-lm"])
    r = run([exe], env=ENV, timeout=300)
    assert "oracle ok" in r.stdout


def test_capi_host_side_under_asan_ubsan(tmp_path):
    hipcc = "/opt/rocm/bin/hipcc" if os.path.exists("/opt/rocm/bin/hipcc") else shutil.which("hipcc")
    if not hipcc:
        pytest.skip("hipcc not found")
    inc = ["-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "libortho_amd", "csrc")]
    san = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
           "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer"]
    objs = []
    for src in (os.path.join(ROOT, "libortho_amd", "csrc", "orth_capi.hip"), os.path.join(SAN, "capi_stubs.hip")):
        obj = str(tmp_path / (os.path.basename(src) + ".o"))
        run([hipcc, "--offload-arch=gfx950", "-O1", "-g", "-fPIC", "-std=c++17", "-Xclang", "-target-feature",
             "-Xclang", "-packed-fp32-ops", *san, *inc, "-c", src, "-o", obj])
        objs.append(obj)
    drv = str(tmp_path / "capi_driver.o")
    run(["gcc", "-O1", "-g", "-std=c11", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
         "-I", os.path.join(ROOT, "include"), "-c", os.path.join(SAN, "capi_driver.c"), "-o", drv])
    exe = str(tmp_path / "capi_san")
    rocm_lib = os.path.join(os.path.dirname(os.path.dirname(os.path.realpath(hipcc))), "lib")
    run(["g++", "-fsanitize=address,undefined", drv, *objs, "-o", exe, "-L", rocm_lib,
         f"-Wl,-rpath,{rocm_lib}", "-lamdhip64", "-lpthread"])
    # no GPU is visible to this process, whatever the host has
    env = dict(ENV, HIP_VISIBLE_DEVICES="-1", ROCR_VISIBLE_DEVICES="-1")
    r = run([exe], env=env, timeout=300)
    assert "capi ok" in r.stdout
