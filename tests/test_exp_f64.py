"""The device's exp restatement (silvic_amd/csrc/exp_f64.hpp, compiled here for the host) equals the C library's
exp bit for bit: the binary-logloss gradients (objective/binary.rs:43) go through it on the device, and silvic's CPU
trainer (and the oracle) through the C library's."""

import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_exp_matches_the_c_library(tmp_path):
    exe = tmp_path / "exp_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-fno-builtin", "-ffp-contract=off", "-o", str(exe),
                    os.path.join(ROOT, "tests", "exp_check.cpp")], check=True)
    out = subprocess.run([str(exe), "4000000"], capture_output=True, text=True, check=True).stdout
    assert int(out.strip()) == 0
