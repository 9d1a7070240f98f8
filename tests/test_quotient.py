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


def _guarded_check(tmp_path, *defines):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    exe = tmp_path / ("guarded_quotient_check" + "".join(d.split("=")[0] for d in defines))
    subprocess.run([gcc, "-O2", "-fopenmp", "-ffp-contract=off", *defines,
                    str(HERE / "native" / "guarded_quotient_check.c"), "-o", str(exe), "-lm"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    return r.returncode, dict(kv.split("=") for kv in r.stdout.split())


@pytest.mark.slow
def test_guarded_quotient_matches_ieee_division(tmp_path):
    """The guarded quotient of smoothed / fp16 / fp32 rows (x * (1 / s), with the IEEE division for
    lanes within 2^-15 of a rounding boundary) and the half-even form of the kernels (the exact product
    rounded by one FMA, guard on fract(fma(x, r, 0.5 + 2^-15)) < 2^-14): no integer differs from the IEEE
    quotient's on 2^28 random (x, absmax) pairs, nor on any fp32 x within 2^-14 of any boundary k + 0.5
    for 2^15 scales s in [1, 2) (~6.9e8 values, of which ~2.3e6 are wrong without the guard)."""
    rc, fields = _guarded_check(tmp_path)
    assert int(fields["samples"]) == 1 << 28
    assert fields["mismatch_even"] == "0" and fields["mismatch_away"] == "0" and fields["mismatch_fma"] == "0"
    assert float(fields["max_gap_ulp"]) <= 4.0
    assert int(fields["sweep_scales"]) == 1 << 15 and int(fields["sweep_values"]) > 600_000_000
    assert fields["sweep_mismatch"] == "0"
    assert int(fields["sweep_hazards"]) > 1_000_000 and int(fields["sweep_hazards_fma"]) > 1_000_000
    assert rc == 0


@pytest.mark.slow
def test_guarded_quotient_check_catches_a_window_below_the_bound(tmp_path):
    """Planted mistake: a 2^-18 window, below the 2^-16 error bound, must make the boundary sweep fail."""
    rc, fields = _guarded_check(tmp_path, "-DWINDOW=0x1p-18f")
    assert int(fields["sweep_mismatch"]) > 0 and rc != 0


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
