"""The packed histogram word's unpacking (silvic_amd/csrc/packed_word.hpp, built here for the host with the
undefined-behaviour sanitizer): every g in -32767..32767 with h on both sides of 32768 comes back exactly, and no
step overflows a signed integer; every small-unit word survives its one-byte code (the split steps' carried
gradients)."""

import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_unpacking_is_exact_and_free_of_signed_overflow(tmp_path):
    exe = tmp_path / "packed_check"
    subprocess.run(["g++", "-O1", "-std=c++17", "-fsanitize=undefined", "-fno-sanitize-recover=all", "-o", str(exe),
                    os.path.join(ROOT, "tests", "packed_check.cpp")], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()
    assert out[0] == "0" and int(out[1]) == 14 * 65535
    assert out[2] == "0" and int(out[3]) == 16 * 15  # every one-byte code of g in -7..7, h in 0..15
