"""The quantizer kernels' fast quotient (reciprocal once per row + one FMA correction) gives the same
int8 as the IEEE fp32 division for every bf16 input, and the row kernels' unclamped half-even rounding
(low byte of v + 1.5 * 2^23) gives the reference's clamped int8 -- proven exhaustively on the CPU
over all ~1.07e9 (x, absmax) bf16 pairs by tests/native/quotient_check.c."""
import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


@pytest.mark.slow
def test_fast_quotient_matches_ieee_division_exhaustively(tmp_path):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    exe = tmp_path / "quotient_check"
    subprocess.run([gcc, "-O2", "-fopenmp", "-ffp-contract=off", str(HERE / "native" / "quotient_check.c"), "-o",
                    str(exe), "-lm"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    fields = dict(kv.split("=") for kv in r.stdout.split())
    assert int(fields["pairs"]) > 1_000_000_000
    assert fields["mismatch_even"] == "0" and fields["mismatch_away"] == "0" and fields["mismatch_magic"] == "0"
    assert float(fields["max_abs_v"]) < 127.5
    assert r.returncode == 0


@pytest.mark.slow
def test_guarded_quotient_matches_ieee_division_sampled(tmp_path):
    """The guarded quotient of smoothed / fp16 / fp32 rows (x * (1 / s), with the IEEE division for
    lanes within 2^-13 of a rounding boundary): 2^28 sampled (x, absmax) pairs, no integer differs from
    the IEEE quotient's, and the product stays within 4 ulps of it (the guard window is 2^-13, at least
    16 ulps for every |x / s| <= 128).  Without the guard the same samples give ~230 mismatches.
    The half-even form of the kernels (the exact product rounded by one FMA, guard on
    fract(fma(x, r, 0.5 + 2^-13)) < 2^-12) is checked on the same samples: no mismatch with its guard,
    274 without it."""
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    exe = tmp_path / "guarded_quotient_check"
    subprocess.run([gcc, "-O2", "-fopenmp", "-ffp-contract=off", str(HERE / "native" / "guarded_quotient_check.c"),
                    "-o", str(exe), "-lm"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    fields = dict(kv.split("=") for kv in r.stdout.split())
    assert int(fields["samples"]) == 1 << 28
    assert fields["mismatch_even"] == "0" and fields["mismatch_away"] == "0" and fields["mismatch_fma"] == "0"
    assert float(fields["max_gap_ulp"]) <= 4.0
    assert r.returncode == 0


def test_one_fma_quantizer_matches_ieee_division_exhaustively(tmp_path):
    """The one-FMA half-even quantizer of the unsmoothed bf16 rows (fma_quant_recip / fma_quant8 in
    mica_amd/csrc/common.h): low byte of fmaf(x, r, 1.5 * 2^23) with the per-row adjusted reciprocal r
    equals clamp(rint(x / s), -127, 127) for all ~1.07e9 (x, absmax) bf16 pairs.  Without the
    adjustment the same check finds 16406 mismatches (x = +-absmax / 2 in 8203 rows)."""
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    exe = tmp_path / "fma_quotient_check"
    subprocess.run([gcc, "-O2", "-fopenmp", "-ffp-contract=off", str(HERE / "native" / "fma_quotient_check.c"), "-o",
                    str(exe), "-lm"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    fields = dict(kv.split("=") for kv in r.stdout.split())
    assert int(fields["pairs"]) > 1_000_000_000
    assert fields["mismatch"] == "0" and int(fields["adjusted_rows"]) > 0
    assert r.returncode == 0
