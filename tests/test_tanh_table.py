"""CPU: the tanh table of csrc/mg_tanh_fast.hpp.

The output tail's fast tanh (and the capped softmax's accepted-rounding path)
expands tanh about the point a0 of one of 128 segments of [0, 1), reading
tanh(a0) from kTanhTab: a0 = 0 for segment 0, (k + 0.5) / 128 for segment k.
The header's table must be exactly what csrc/gen_tanh_table.py prints (no hand
edits), and each entry must be tanh at its segment's point: checked against
libm's tanh, an independent evaluation, within 2 ulp.
"""
import math
import pathlib
import re
import subprocess
import sys

ROOT = pathlib.Path(__file__).resolve().parents[1]
CSRC = ROOT / "muse-glimmer-intel-serve_amd" / "csrc"
HEX = re.compile(r"-?0x[0-9a-fA-F.]+p[-+]?\d+")


def table_of(text):
    body = text[text.index("kTanhTab[128] = {"):]
    body = body[:body.index("};")]
    return [float.fromhex(t) for t in HEX.findall(body)]


def test_header_table_is_the_generator_output():
    out = subprocess.run([sys.executable, str(CSRC / "gen_tanh_table.py")], check=True, capture_output=True,
                         text=True).stdout
    assert table_of((CSRC / "mg_tanh_fast.hpp").read_text()) == table_of(out)


def test_table_entries_are_tanh_of_the_segment_points():
    tab = table_of((CSRC / "mg_tanh_fast.hpp").read_text())
    assert len(tab) == 128
    assert tab[0] == 0.0  # segment 0 is taken about 0
    for k in range(1, 128):
        ref = math.tanh((k + 0.5) / 128)
        assert abs(tab[k] - ref) <= 2 * math.ulp(ref), k
        # a wrong centre (k / 128 or (k + 1) / 128) is off by far more
        assert abs(tab[k] - math.tanh(k / 128)) > 1e-4
