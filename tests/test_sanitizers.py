"""The CPU codec (astc-kv_amd/csrc/codec) and the oracle's C decoder built
with AddressSanitizer and UndefinedBehaviorSanitizer (g++ / gcc, host code
only) and driven through every codec entry point by
tests/sanitize/codec_sanitize.cpp: random blocks of eleven footprints (up to 64 texels; larger ones are refused)
against the oracle, block classes, encode/decode round trips of images with
partial edge blocks, and the short-buffer refusals. Any sanitizer report
aborts the run."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CODEC = ROOT / "astc-kv_amd" / "csrc" / "codec"
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]


@pytest.mark.skipif(shutil.which("g++") is None or shutil.which("gcc") is None, reason="needs gcc/g++")
def test_codec_and_oracle_under_asan_ubsan(tmp_path):
    obj = tmp_path / "oracle.o"
    subprocess.run(["gcc", "-std=c11", *SAN, "-c", str(ROOT / "oracle" / "astc_oracle.c"), "-o", str(obj)],
                   check=True)
    exe = tmp_path / "codec_sanitize"
    srcs = [CODEC / s for s in ("astc_format.cpp", "astc_decode.cpp", "astc_encode.cpp", "bridge.cpp")]
    subprocess.run(["g++", "-std=c++17", *SAN, "-ffp-contract=off", f"-I{ROOT / 'include'}", f"-I{CODEC}",
                    str(ROOT / "tests" / "sanitize" / "codec_sanitize.cpp"), *map(str, srcs), str(obj),
                    "-o", str(exe), "-lm", "-lpthread"], check=True)
    r = subprocess.run([str(exe), "20000"], capture_output=True, text=True, timeout=600,
                       env={"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=1", "UBSAN_OPTIONS": "print_stacktrace=1"})
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 problems" in r.stdout
