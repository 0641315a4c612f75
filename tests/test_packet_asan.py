"""The store reader (host_packet.cpp) under AddressSanitizer and
UndefinedBehaviorSanitizer on the CPU: tests/asan_packet.cpp feeds it the
compiled 4-layer store (oracle/make_c1.sh) and damaged copies - flipped header
and drive-list bytes, truncations, hostile packet records with the table's
SHA-256 and header CRC recomputed, damaged tensor directories - and every one
must load or be refused without a sanitizer report.  CPU only."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
C1 = os.path.join(ROOT, "oracle", "_ref", "c1", "c1.tlmm")


@pytest.mark.skipif(not os.path.exists(C1), reason="oracle/_ref/c1 not built (oracle/make_c1.sh)")
@pytest.mark.skipif(shutil.which("g++") is None, reason="no g++")
def test_store_reader_under_asan_ubsan(tmp_path):
    exe = tmp_path / "asan_packet"
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                    "-fno-omit-frame-pointer", os.path.join(ROOT, "tests", "asan_packet.cpp"),
                    os.path.join(ROOT, "tierlm_amd", "csrc", "host_packet.cpp"), "-o", str(exe)], check=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([str(exe), C1, str(tmp_path)], capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, r.stderr[-4000:]
    assert "asan_packet: done" in r.stdout
