"""The C ABI's host side under AddressSanitizer, on the CPU.

The library's sources are compiled with the host pass instrumented
(``-Xarch_host -fsanitize=address``; device code is built as usual and never
runs here), linked with ``capi_asan_driver.cpp`` and run: argument
validation of every entry point, workspace sizing, and the host path of
well-formed calls up to their launch (which fails without a GPU).  A heap or
stack overrun, a use after free or a double free in the host code aborts the
run with a sanitizer report.  No GPU is used.
"""
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
sys.path.insert(0, os.path.join(REPO, "aoa-kv_amd", "aoakv"))


def _flags():
    import _build as B
    f = [x for x in B.FLAGS if x not in ("-O3", "-Wall")]
    return B, f + ["-O1", "-g", "-Xarch_host", "-fsanitize=address",
                   "-Xarch_host", "-fno-omit-frame-pointer"]


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    B, flags = _flags()
    if not os.path.exists(B.HIPCC) or shutil.which("g++") is None:
        pytest.skip("hipcc or g++ missing")
    out = tmp_path_factory.mktemp("capi_asan")

    def comp(src):
        obj = str(out / (os.path.splitext(src)[0] + ".o"))
        cmd = [B.HIPCC, *flags, "-x", "hip", "-c", os.path.join(B.SRC_DIR, src), "-o", obj]
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-3000:]
        return obj

    with cf.ThreadPoolExecutor(max_workers=6) as ex:
        objs = list(ex.map(comp, B.SOURCES))
    drv = str(out / "driver.o")
    r = subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address",
                        "-fno-omit-frame-pointer", "-c",
                        os.path.join(HERE, "capi_asan_driver.cpp"), "-o", drv],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    exe = str(out / "capi_asan_driver")
    r = subprocess.run([B.HIPCC, f"--offload-arch={B.ARCH}", "-Xarch_host", "-fsanitize=address",
                        *objs, drv, "-o", exe], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    return exe


def test_driver_is_instrumented(driver):
    nm = subprocess.run(["nm", driver], capture_output=True, text=True).stdout
    assert "__asan_report_load" in nm or "__asan_init" in nm


def test_c_abi_host_side_under_asan(driver):
    env = dict(os.environ)
    # the HIP runtime's own allocations at exit are not the library's
    env["ASAN_OPTIONS"] = "detect_leaks=0:halt_on_error=1:abort_on_error=0"
    # no device for the runtime to find here; keep it off any GPU elsewhere
    env["HIP_VISIBLE_DEVICES"] = ""
    r = subprocess.run([driver], capture_output=True, text=True, env=env, timeout=300)
    log = r.stdout + r.stderr
    assert "AddressSanitizer" not in log, log[-4000:]
    assert r.returncode == 0, log[-4000:]
    assert "0 failures" in r.stdout
