"""The oracle under AddressSanitizer and UndefinedBehaviorSanitizer.

The reference runs `go test -race ./...` in CI (reference
.github/workflows/ci.yml:40-41); the counterpart here for the C code is a
sanitizer build. oracle/mimref.c is built once more with
-fsanitize=address,undefined (no recovery: the first finding aborts), and
the oracle's own tests run against it through MIMREF_LIB in a subprocess
with the ASan runtime preloaded (Python itself is not instrumented). Any
out-of-bounds access, overflow or other undefined behaviour in the
decoders, the quantizer, the dot products, the float32 paths and the
decoder ops fails the run. CPU only."""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _asan_runtime():
    out = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True)
    path = out.stdout.strip()
    return path if os.path.isabs(path) and os.path.exists(path) else None


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_oracle_tests_pass_under_asan_and_ubsan(tmp_path):
    rt = _asan_runtime()
    if rt is None:
        pytest.skip("gcc has no AddressSanitizer runtime here")
    lib = tmp_path / "libmimref_san.so"
    cmd = ["gcc", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=all", "-mavx2", "-mfma", "-ffp-contract=off", "-fPIC", "-fopenmp", "-std=c11",
           "-shared", "-o", str(lib), os.path.join(ROOT, "oracle", "mimref.c"), "-lm"]
    subprocess.run(cmd, check=True, capture_output=True)
    env = dict(os.environ, MIMREF_LIB=str(lib), LD_PRELOAD=rt,
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")
    tests = [os.path.join(ROOT, "tests", t) for t in ("test_oracle.py", "test_oracle_decoder.py", "test_quant_rne.py")]
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider", "-m", "not gpu", *tests],
                       env=env, capture_output=True, text=True, timeout=900)
    tail = (r.stdout + r.stderr)[-4000:]
    assert r.returncode == 0, tail
    assert "AddressSanitizer" not in tail and "runtime error" not in tail, tail
