"""The paired f32 -> bf16 conversion the GEMV stagings split activations with (gfx950's
v_cvt_pk_bf16_f32, mx_device.hpp f32x2_to_bf16x2_bits) against the library's integer rounding
(f32_to_bf16_bits: nearest even, quiet NaN) on every one of the 2^32 f32 inputs, both halves of the
pair: tests/native/bf16_convert_check.hip, built with the library."""
import pathlib
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
EXE = ROOT / "burn-extended_amd" / "lib" / "checks" / "bf16_convert_check"


@pytest.mark.gpu
def test_bf16_pair_convert_matches_integer_rounding_everywhere():
    assert EXE.exists(), f"{EXE} is not built; run __graft_entry__.build()"
    print("[convert] exhaustive bf16 pair conversion check", flush=True)
    r = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=90)
    print(r.stdout.strip(), r.stderr.strip(), flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches non-NaN 0 NaN 0" in r.stdout
