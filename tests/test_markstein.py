"""The pack kernel's division-free quotient equals IEEE division on the codec's domain.

The kernel computes rint((x - min) / scale) with Markstein's correction of a * RN(1/b)
(three float ops per element instead of a division); ``markstein_check.c`` compares the
two bit for bit: every dividend of eight divisors with extreme mantissas, plus random
dividends for random divisors and for span/15 scales.  CPU only.
"""
import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_markstein_quotient_is_the_ieee_quotient(tmp_path):
    exe = tmp_path / "markstein_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), str(HERE / "markstein_check.c"), "-lm"],
                   check=True)
    out = subprocess.run([str(exe), "20000", "300"], capture_output=True, text=True, timeout=600)
    print(out.stdout)
    assert out.returncode == 0, out.stdout
    assert " 0 differ" in out.stdout
