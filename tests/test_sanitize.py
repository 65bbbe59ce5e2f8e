"""Host-side sanitizer builds (no GPU): the safetensors/JSON reader of the C
ABI fuzzed under AddressSanitizer + UndefinedBehaviorSanitizer, and the
oracle run at its buffer limits under the same.  Built with g++/gcc on the
host code only (no .hip file is compiled here)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]


def build_and_run(tmp_path, compiler, sources, extra=()):
    if shutil.which(compiler) is None:
        pytest.skip(f"{compiler} not available")
    exe = str(tmp_path / "prog")
    subprocess.run([compiler, *SAN, *extra, *sources, "-o", exe, "-lm", "-pthread"], check=True,
                   capture_output=True, timeout=300)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    return subprocess.run([exe], capture_output=True, text=True, timeout=300, env=env)


def test_safetensors_reader_fuzz_asan_ubsan(tmp_path):
    r = build_and_run(tmp_path, "g++", [os.path.join(ROOT, "teenygrad_amd", "csrc", "safetensors.cpp"),
                                         os.path.join(ROOT, "tests", "native", "st_fuzz.cpp")], ["-std=c++17"])
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr
    assert "accepted" in r.stdout


def test_oracle_bounds_asan_ubsan(tmp_path):
    r = build_and_run(tmp_path, "gcc", [os.path.join(ROOT, "oracle", "teeny_oracle.c"),
                                         os.path.join(ROOT, "tests", "native", "oracle_bounds.c")], ["-std=c11"])
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr
    assert "oracle bounds: ok" in r.stdout
