"""The reciprocal-corrected quotient used by the beam kernel equals IEEE division
(tests/division_check.c), so the kernel's candidate errors stay bit-identical to the
reference's `s / R(i,i)` (src/quantizer/beam_search.cpp:146, :160)."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))


def test_reciprocal_corrected_quotient_is_ieee(tmp_path):
    exe = str(tmp_path / "division_check")
    subprocess.run(["gcc", "-O2", "-mfma", "-ffp-contract=off", "-fopenmp",
                    os.path.join(HERE, "division_check.c"), "-o", exe, "-lm"], check=True)
    res = subprocess.run([exe, "48", "20000000"], capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "mismatches=0" in res.stdout
