"""The library's host code under AddressSanitizer and UndefinedBehaviorSanitizer.

Every source is compiled with the sanitizers on its host compilation only
(`-Xarch_host`), linked into a shared library, and driven by
`tests/host_abi_driver.cpp`: the argument checks, workspace sizes, path and
layout queries of every entry point, all of which return before a launch (no
kernel runs).  Runs on the CPU.
"""

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "latent_amd" / "csrc"
HIPCC = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
CLANGXX = str(Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "llvm" / "bin" / "clang++")

# Sanitizers apply to the host compilation only (-Xarch_host before each).
SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
       "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer"]
# Device code is compiled as for the library (the host side refers to its
# code object) but never loaded: nothing here launches a kernel.
COMMON = ["-O1", "-g", "-std=c++17", "--offload-arch=gfx950", "-Xarch_device", "-O3", "-Xarch_device", "-g0",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-fPIC", "-munsafe-fp-atomics",
          "-Wno-unused-command-line-argument"]


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    if not Path(HIPCC).exists() or not Path(CLANGXX).exists():
        pytest.skip("hipcc / clang++ not found")
    out = tmp_path_factory.mktemp("san")
    sources = sorted(CSRC.glob("*.hip"))
    cmds = [[HIPCC, *COMMON, *SAN, "-c", str(s), "-o", str(out / (s.stem + ".o"))] for s in sources]
    with ThreadPoolExecutor(max_workers=min(8, len(cmds))) as pool:
        for r in pool.map(lambda c: subprocess.run(c, capture_output=True, text=True), cmds):
            assert r.returncode == 0, r.stderr[-3000:]
    lib = out / "liblatent_hip_san.so"
    r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *SAN,
                        *[str(out / (s.stem + ".o")) for s in sources], "-o", str(lib)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    # The driver is plain C++: the ROCm clang++ (the compiler behind hipcc, so
    # one sanitizer runtime serves both) builds it and links the runtime in.
    exe = out / "host_abi_driver"
    r = subprocess.run([CLANGXX, "-O1", "-g", "-std=c++17", *SAN, "-I", str(ROOT / "include"),
                        str(ROOT / "tests" / "host_abi_driver.cpp"), str(lib), f"-Wl,-rpath,{out}", "-o", str(exe)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    return exe


def test_host_entry_points_are_clean_under_asan_and_ubsan(driver):
    env = dict(os.environ)
    # The HIP runtime's own allocations are not this library's to check, and
    # the environment's preloaded libraries stay as they are (the link-order
    # check would otherwise refuse to start under them).
    env["ASAN_OPTIONS"] = "detect_leaks=0:halt_on_error=1:abort_on_error=0:verify_asan_link_order=0"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    r = subprocess.run([str(driver)], capture_output=True, text=True, env=env, timeout=300)
    log = r.stdout + r.stderr
    assert "AddressSanitizer" not in log and "runtime error" not in log, log[-4000:]
    assert r.returncode == 0, log[-4000:]
    assert "host ABI checks: 0 failed" in r.stdout
