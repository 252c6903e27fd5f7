"""AddressSanitizer / UndefinedBehaviorSanitizer and ThreadSanitizer builds of
the oracle and of libg3attn's host code, run on the CPU.

oracle/Makefile `san` builds oracle/_san/san_check (oracle/san_check.c) with
-fsanitize=address,undefined over g3_oracle.c, host/g3attn.c,
host/rope_table.c and backend/g3backend.c (gcc; the HIP kernel objects are
linked as built and never launched).  `tsan` builds the oracle part alone
with -fsanitize=thread, for its threaded prefill and generator.  Both stop at
the first report (-fno-sanitize-recover=all, halt_on_error) and also check
their own results, so a clean exit means: no memory error, no undefined
behaviour, no data race and no wrong answer on the driven paths.  A canary
with a planted heap overflow shows the sanitizer is live in this toolchain.
"""
import os
import shutil
import subprocess

import pytest

from helpers import REPO

ORACLE = os.path.join(REPO, "oracle")
SAN = os.path.join(ORACLE, "_san")

pytestmark = pytest.mark.skipif(not shutil.which("gcc"), reason="gcc not available")


@pytest.fixture(scope="module")
def built():
    r = subprocess.run(["make", "-C", ORACLE, "san", "tsan"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    return True


def _run(exe, env_extra, args=()):
    env = dict(os.environ, **env_extra)
    env.pop("G3ATTN_FAULT", None)
    return subprocess.run([os.path.join(SAN, exe), *args], capture_output=True, text=True, timeout=600, env=env)


def test_asan_ubsan_oracle_and_host(built):
    args = ("--gpu-present",) if os.path.exists("/dev/kfd") else ()
    r = _run("san_check", {"ASAN_OPTIONS": "detect_leaks=1", "UBSAN_OPTIONS": "print_stacktrace=1"}, args)
    assert r.returncode == 0 and "san_check: ok" in r.stdout, r.stderr[-4000:]
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr


def test_tsan_oracle_threads(built):
    r = _run("tsan_check", {"TSAN_OPTIONS": "halt_on_error=1"})
    assert r.returncode == 0 and "san_check: ok" in r.stdout, r.stderr[-4000:]
    assert "ThreadSanitizer" not in r.stderr


def test_sanitizer_catches_a_planted_overflow(tmp_path):
    src = tmp_path / "canary.c"
    src.write_text("#include <stdlib.h>\n"
                   "int main(int c, char **v) { (void)v; int *a = malloc(4 * sizeof(int));"
                   " int x = a[c + 3]; free(a); return x & 0; }\n")
    exe = tmp_path / "canary"
    subprocess.run(["gcc", "-g", "-O0", "-fsanitize=address", "-o", str(exe), str(src)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode != 0 and "heap-buffer-overflow" in r.stderr
