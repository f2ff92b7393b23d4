"""The library's host C under AddressSanitizer and UndefinedBehaviorSanitizer,
the counterpart of the reference's `make san` (Makefile:140-159, its whole
suite under ASan + UBSan). CPU only.

tests/fakehip builds the library's C sources (the shim, the decode host, the
GGUF reader, the dispatch table) against its HIP stand-in a second time with
-fsanitize=address,undefined -fno-sanitize-recover=all, so that every report
ends the process. In a child process that preloads gcc's ASan runtime:

  * the failure-injection suite (every HIP call of every entry point failing
    in turn) and the GGUF suite (71 images, statuses against the reference's
    own reader) run against that build;
  * tests/gguf_fuzz.py mutates those images (bit flips, edge values, cuts,
    splices, mostly in the header) and reads each mutant, copied into a
    buffer of exactly its size from the C allocator, for a bounded time.

Either must exit 0 with no sanitizer report in its output.
"""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FAKE_DIR = os.path.join(ROOT, "tests", "fakehip")
SAN_LIB = os.path.join(FAKE_DIR, "libsllm_gfx950_fakehip_san.so")
FUZZ_SECONDS = 30


def _asan_runtime():
    r = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True)
    path = r.stdout.strip()
    return path if r.returncode == 0 and os.path.isabs(path) and os.path.exists(path) else None


@pytest.fixture(scope="module")
def san_env():
    asan = _asan_runtime()
    if asan is None:
        pytest.skip("gcc's AddressSanitizer runtime is not installed")
    r = subprocess.run(["make", "-s", "-C", FAKE_DIR, "libsllm_gfx950_fakehip_san.so"], capture_output=True, text=True)
    if r.returncode != 0:
        pytest.fail(f"building the sanitizer library failed:\n{r.stdout}\n{r.stderr}")
    env = dict(os.environ)
    env["LD_PRELOAD"] = asan + (":" + env["LD_PRELOAD"] if env.get("LD_PRELOAD") else "")
    # Python itself is not instrumented and keeps its objects to exit: no leak report
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1:detect_stack_use_after_return=1"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    env["SLLM_FAKEHIP_SAN"] = "1"
    env["SLLM_TEST_LIB"] = SAN_LIB
    return env


def _clean(r):
    out = r.stdout + r.stderr
    assert "AddressSanitizer" not in out and "runtime error:" not in out, out[-6000:]
    assert r.returncode == 0, out[-6000:]
    return out


def test_failure_paths_and_gguf_reader_under_asan_and_ubsan(san_env):
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider", "-m", "not gpu",
                        os.path.join(ROOT, "tests", "test_failure_injection.py"),
                        os.path.join(ROOT, "tests", "test_gguf_load.py")],
                       cwd=ROOT, env=san_env, capture_output=True, text=True, timeout=900)
    out = _clean(r)
    assert " passed" in out and " failed" not in out


def test_gguf_reader_mutation_fuzz_under_asan_and_ubsan(san_env):
    r = subprocess.run([sys.executable, os.path.join(ROOT, "tests", "gguf_fuzz.py"), SAN_LIB, str(FUZZ_SECONDS), "7"],
                       cwd=ROOT, env=san_env, capture_output=True, text=True, timeout=300)
    out = _clean(r)
    assert "no finding" in out, out[-3000:]


def test_the_sanitizer_build_reports_a_read_past_the_image(san_env):
    """The plumbing itself: a 16-byte buffer (magic, version 3, the tensor
    count) handed over as 1000 bytes must end the child with an
    AddressSanitizer report: the reader's next read, the metadata count at
    bytes 16..23, lies past the buffer."""
    code = ("import ctypes, sys; L = ctypes.CDLL(sys.argv[1]); libc = ctypes.CDLL(None);"
            "libc.malloc.restype = ctypes.c_void_p; b = libc.malloc(16); ctypes.memmove(b, b'GGUF' + (3).to_bytes(4, 'little') + bytes(8), 16);"
            "d = ctypes.create_string_buffer(4096); t = ctypes.create_string_buffer(1 << 16);"
            "L.sllm_gfx950_gguf_describe(ctypes.c_void_p(b), ctypes.c_size_t(1000), d, t)")
    r = subprocess.run([sys.executable, "-c", code, SAN_LIB], cwd=ROOT, env=san_env, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode != 0 and "AddressSanitizer: heap-buffer-overflow" in r.stderr, r.stderr[-3000:]
