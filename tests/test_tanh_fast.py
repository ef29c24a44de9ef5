"""CPU: exhaustive check of the output tail's fast tanh.

The vocab pass applies rnd(tanh(v)) to every logit when the output tail is on
(src/muse_glimmer.hpp:920-943). The device evaluates a short f64 tanh
(csrc/mg_tanh_fast.hpp) and accepts its rounding only when the whole error
interval rounds to one stored value, falling back to FDLIBM otherwise. That
is exact only if the fast value's error is inside the interval for every
input. tanh is only ever applied to stored values (f32, bf16, f16 — all of
them floats), so running every float below 22 through both functions (the
same plain C++ the device compiles, and the oracle's FDLIBM restatement)
proves it: no accepted rounding may differ, and the error must stay well
below the margin.
"""
import pathlib
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = tmp_path_factory.mktemp("tanh") / "tanh_fast_check"
    subprocess.run(["g++", "-std=c++20", "-O2", "-fopenmp", "-ffp-contract=off", "-march=x86-64-v3",
                    f"-I{ROOT / 'muse-glimmer-intel-serve_amd' / 'csrc'}", f"-I{ROOT / 'oracle'}",
                    str(ROOT / "tests" / "host" / "tanh_fast_check.cpp"), "-o", str(exe)], check=True)
    return exe


def run(exe, stride, margin=None, perturb=None):
    args = [str(exe), str(stride)] + ([repr(margin)] if margin is not None else [])
    args += [repr(perturb)] if perturb is not None else []
    out = subprocess.run(args, check=True, capture_output=True, text=True).stdout.split()
    maxrel, bad, fb32, fbb, fbh, count = float(out[0]), *map(int, out[1:])
    return maxrel, bad, fb32, fbb, fbh, count


def test_every_float_below_22(checker):
    maxrel, bad, fb32, fbb, fbh, count = run(checker, 1)
    assert count == 0x41B00000
    assert bad == 0
    assert maxrel < 2.0**-40 / 16          # the margin holds with 16x to spare
    assert fb32 < count * 1e-5 and fbb < count * 1e-5 and fbh < count * 1e-5


def test_the_check_has_teeth(checker):
    """a fast value off by 2^-34 (planted on the CPU) is caught: without a margin
    and with a margin smaller than that error, some accepted roundings differ
    from FDLIBM's; a margin above it accepts none wrongly"""
    maxrel, bad, fb32, _, _, count = run(checker, 1, 0.0, 2.0**-34)
    assert bad > 0 and fb32 == 0 and maxrel > 2.0**-35
    _, bad, _, _, _, _ = run(checker, 1, 2.0**-40, 2.0**-34)
    assert bad > 0
    _, bad, _, _, _, _ = run(checker, 1, 2.0**-33, 2.0**-34)
    assert bad == 0
