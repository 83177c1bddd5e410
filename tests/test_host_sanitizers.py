"""The host libraries (the g_vbs_hip_backend shim with the decode driver and
the synthetic generator, and the CPU hot-kernel module) under AddressSanitizer
and UBSan: `make sanitize` builds them into lib-san/ with gcc, and the CPU
suite runs again in a child process that preloads the sanitizer runtimes and
loads those builds through VBS_GFX950_HOST_LIB_DIR. UBSan is built
non-recovering, so any report fails the child; ASan stops at its first
report. Leak checking is off (the Python interpreter itself is not built for
it). The full-size 7B oracle check is left out: it exercises the synthetic
generator at a size the sanitizer makes slow, and the small models cover the
same code."""
import os
import subprocess
import sys

import pytest

import vbs_gfx950 as V

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "verum-bespoke-singularity_amd")
SAN_DIR = os.path.join(PKG, "lib-san")


def runtime(name):
    p = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True)
    path = p.stdout.strip()
    return path if os.path.isabs(path) and os.path.exists(path) else None


@pytest.fixture(scope="module")
def san_env():
    asan, ubsan = runtime("libasan.so"), runtime("libubsan.so")
    if not (asan and ubsan):
        pytest.skip("gcc's sanitizer runtimes are not installed here")
    subprocess.run(["make", "-s", "-C", PKG, "sanitize"], check=True)
    env = dict(os.environ)
    env.update(LD_PRELOAD=f"{asan} {ubsan}",
               ASAN_OPTIONS="detect_leaks=0:verify_asan_link_order=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1",
               VBS_GFX950_HOST_LIB_DIR=SAN_DIR, PYTHONDONTWRITEBYTECODE="1")
    return env


def test_sanitized_builds_are_the_ones_loaded(san_env):
    code = ("import sys; sys.path.insert(0, %r); import vbs_gfx950 as V, ctypes as C; "
            "V.load_host(); C.CDLL(V.HOT_LIB); "
            "maps = open('/proc/self/maps').read(); "
            "print(%r in maps, 'libasan' in maps, 'libubsan' in maps)" % (PKG, SAN_DIR))
    p = subprocess.run([sys.executable, "-c", code], env=san_env, capture_output=True, text=True,
                       timeout=120)
    assert p.returncode == 0, p.stderr[-2000:]
    assert p.stdout.split() == ["True", "True", "True"], p.stdout
    assert V.HOST_LIB.startswith(V.LIB_DIR)  # this process keeps the normal build


def test_cpu_suite_under_asan_and_ubsan(san_env):
    tests = [os.path.join(ROOT, "tests", f) for f in sorted(os.listdir(os.path.join(ROOT, "tests")))
             if f.startswith("test_") and f.endswith(".py") and f != os.path.basename(__file__)]
    p = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-m", "not gpu", "-k", "not 7b",
                        "-p", "no:cacheprovider", *tests], env=san_env, capture_output=True,
                       text=True, timeout=1200, cwd=ROOT)
    out = p.stdout + p.stderr
    assert p.returncode == 0, out[-4000:]
    assert "runtime error" not in out and "AddressSanitizer" not in out, out[-4000:]
    assert " passed" in out
