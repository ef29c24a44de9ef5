"""CPU: exhaustive checks of the softmax kernel's capped score
(csrc/mg_softcap_fast.hpp), which the fast softmax path uses for softcap rows.

It replaces the IEEE division s / cap by Markstein's correction with a
host-rounded reciprocal, and FDLIBM's tanh by the f64 series of tanh_fast_abs
whose f32 rounding is accepted only when a bit test on the mantissa shows it
certain. Both are exact only if they hold for every input they accept, so the
checker (tests/host/softcap_fast_check.cpp, the same plain C++ the device
compiles) runs every input: every normal-range f32 quotient at several caps,
every float in [2^-100, 2^-5) through the rounding test against the oracle's
FDLIBM tanh, and the whole capped score against the twin's chain (each step
exact in f64, rounded to f32) on a strided sweep of all f32 scores, for caps in
the range the kernel uses it for (1 <= |cap| <= 2^20, negative caps included),
with the reciprocal the kernels are given (recip_rn).
"""
import pathlib
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = tmp_path_factory.mktemp("softcap") / "softcap_fast_check"
    subprocess.run(["g++", "-std=c++20", "-O2", "-fopenmp", "-ffp-contract=off", "-march=x86-64-v3",
                    f"-I{ROOT / 'muse-glimmer-intel-serve_amd' / 'csrc'}", f"-I{ROOT / 'oracle'}",
                    str(ROOT / "tests" / "host" / "softcap_fast_check.cpp"), "-o", str(exe)], check=True)
    return exe


def run(exe, *args):
    out = subprocess.run([str(exe), *map(str, args)], check=True, capture_output=True, text=True).stdout
    return [float(v) if "." in v or "e" in v else int(v) for v in out.split()]


@pytest.mark.parametrize("cap", ("30", "50", "20", "1", "3", "7.5", "0.7", "0.001", "12345.678", "1048575.9",
                                 "1048576", "-30", "-1", "-1048576"))
def test_markstein_quotient_is_correctly_rounded(checker, cap):
    bad, count = run(checker, "quot", cap)
    assert count == 0x71800000 - 0x0d800000 - 1
    assert bad == 0


def test_series_rounding_test_accepts_only_fdlibm_roundings(checker):
    bad, fb, count, maxrel = run(checker, "tanh", 0x2000)
    assert count == 0x3d000000 - 0x0d800000
    assert bad == 0
    assert maxrel < 2.0**-45                # the 2^-40 margin holds with 32x to spare
    assert fb < count * 1e-5


def test_rounding_test_sees_errors_beyond_its_margin(checker):
    """a planted 2^-30 relative error in the series value (beyond the 2^-40
    margin) makes accepted roundings differ from FDLIBM's"""
    bad, _, _, _ = run(checker, "tanh", 0x2000, repr(2.0**-30))
    assert bad > 0


@pytest.mark.parametrize("scale,cap", (("0.08838834764831845", "30"), ("1.0", "50"), ("0.125", "20"), ("2.0", "1"),
                                       ("0.08838834764831845", "-30"), ("1.0", "1048576")))
def test_capped_score_equals_the_twin(checker, scale, cap):
    bad, fb, count = run(checker, "score", scale, cap, 7)
    assert bad == 0
    assert count > 600_000_000 and fb < count
