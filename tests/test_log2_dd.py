"""The device's lambdarank normalization factor rests on log2_bracket (silvic_amd/csrc/log2_dd.hpp): the two doubles
around log2(x) from a double-double evaluation. Built here for the host with -ffp-contract=off, as the device build
is, and checked two ways: against log2 to 50 significant digits (Python's decimal module), which the bracket must
enclose with its two ends one double apart, and against the C library's log2 (what silvic's f64::log2 calls), which
must be one of the two ends (or the value itself when it is a double) on every input. A bracket that dropped the
low half of 1/ln 2 or one of the leading series terms would miss the decimal values."""

import math
import os
import random
import subprocess
from decimal import Decimal, getcontext

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def exe(tmp_path_factory):
    out = tmp_path_factory.mktemp("log2") / "log2_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-o", str(out),
                    os.path.join(ROOT, "tests", "log2_check.cpp")], check=True)
    return str(out)


def _inputs(seed, n):
    rnd = random.Random(seed)
    xs = [1.0, 2.0, 3.0, 1.5, math.nextafter(1.0, 2.0), math.nextafter(2.0, 0.0), math.nextafter(2.0, 4.0), 2.0 ** 40,
          1.0 + 2.0 ** -52, 1.0 + 2.0 ** -30, 1.4142135623730951, 1.4142135623730950, 0.75 * 2 ** 20]
    for _ in range(n):
        xs.append(1.0 + 2.0 ** rnd.uniform(-60, 40))
    return xs


def test_bracket_encloses_the_exact_logarithm(exe):
    xs = _inputs(3, 3000)
    res = subprocess.run([exe, "dump"], input="\n".join(x.hex() for x in xs), capture_output=True, text=True,
                         check=True).stdout.split("\n")
    getcontext().prec = 50
    ln2 = Decimal(2).ln()
    checked = 0
    for x, line in zip(xs, res):
        xs_, lo_, hi_, st = line.split()
        assert float.fromhex(xs_) == x
        lo, hi, st = float.fromhex(lo_), float.fromhex(hi_), int(st)
        k = round(math.log2(x))
        if x == 2.0 ** k:  # a power of two: the logarithm is the exponent, a double
            assert st == 0 and lo == hi == float(k)
            continue
        exact = Decimal(x).ln() / ln2
        assert st == 1, x
        assert Decimal(lo) < exact < Decimal(hi), (x, lo, hi)
        assert math.nextafter(lo, math.inf) == hi
        checked += 1
    assert checked >= 2500  # the rest are powers of two (1 + s rounds to 1 for s below 2^-53)


def test_the_series_reciprocals_are_the_fma_residual_pairs(exe):
    # the table's pairs (written from decimal arithmetic) equal what an fma residual gives: hi = 1/k rounded, lo the
    # rounded rest
    assert subprocess.run([exe, "table"], capture_output=True, text=True, check=True).stdout.split() == ["0"]


def test_the_c_library_log2_is_an_end_of_the_bracket(exe):
    bad, undecided, n = map(int, subprocess.run([exe, "glibc", "4000000", "11"], capture_output=True, text=True,
                                                check=True).stdout.split())
    assert n == 4000000 and bad == 0 and undecided == 0
