"""The host side of the C ABI under AddressSanitizer (CPU; no GPU needed).

Every library source is compiled with its host pass instrumented (the device code is built
as usual and never runs), linked with ``tests/asan/host_abi_driver.cpp``, and run: plans,
workspace sizes and argument validation with ordinary, edge-case and invalid inputs, all of
which return before any HIP launch. A memory error ends the driver with ASan's report.
"""
import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(ROOT, "xnn_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"
# the instrumentation applies to the host pass only
SAN = ["-Xarch_host -fsanitize=address", "-fno-omit-frame-pointer"]


def _hipcc_ok() -> bool:
    return os.path.exists(HIPCC)


@pytest.mark.skipif(not _hipcc_ok(), reason="hipcc is not installed")
def test_host_abi_under_address_sanitizer(tmp_path):
    from xnn_amd.build import SOURCES
    flags = ["-O1", "-g", "-std=c++17", "-fPIC", "--offload-arch=gfx950",
             "-Wno-unused-result", "-Wno-unused-command-line-argument",
             "-I", os.path.join(ROOT, "include"), "-I", CSRC]

    def compile_one(name):
        obj = str(tmp_path / name.replace(".hip", ".o"))
        cmd = " ".join([HIPCC, *flags, *SAN, "-c", os.path.join(CSRC, name), "-o", obj])
        res = subprocess.run(cmd, shell=True, capture_output=True, text=True)
        assert res.returncode == 0, f"{name}: {res.stderr[-3000:]}"
        return obj

    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as pool:
        objs = list(pool.map(compile_one, SOURCES))
    driver = str(tmp_path / "host_abi_driver.o")
    cmd = " ".join([HIPCC, "-x", "c++", "-O1", "-g", "-std=c++17", *SAN, "-I",
                    os.path.join(ROOT, "include"), "-c",
                    os.path.join(HERE, "asan", "host_abi_driver.cpp"), "-o", driver])
    res = subprocess.run(cmd, shell=True, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-3000:]
    exe = str(tmp_path / "host_abi_driver")
    cmd = " ".join([HIPCC, *SAN, driver, *objs, "-o", exe])
    res = subprocess.run(cmd, shell=True, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-3000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0", HIP_VISIBLE_DEVICES="")
    run = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=120)
    out = run.stdout + run.stderr
    assert "AddressSanitizer" not in out, out[-4000:]
    assert run.returncode == 0 and "host ABI checks passed" in run.stdout, out[-4000:]
