"""The device arithmetic of the codec (csrc/codec_math.h), compiled for the host
and compared exhaustively with IEEE division and std::lround.

The kernels replace `a / b` by a reciprocal multiply with one fma correction
and `lround` by a truncating add; these tests are what licenses that."""

import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SOURCE = ROOT / "tests" / "codec_math_check.cpp"
CSRC = ROOT / "gdn-state-codec_amd" / "csrc"


def _has_fma() -> bool:
    try:
        return " fma " in Path("/proc/cpuinfo").read_text().replace("\n", " ")
    except OSError:
        return False


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    if not _has_fma():
        pytest.skip("host CPU has no FMA; the software fmaf is too slow for these sweeps")
    binary = tmp_path_factory.mktemp("codec_math") / "codec_math_check"
    subprocess.run(
        ["g++", "-std=c++17", "-O2", "-mfma", "-ffp-contract=off", "-fno-fast-math",
         "-pthread", f"-I{CSRC}", str(SOURCE), "-o", str(binary)],
        check=True,
    )
    return binary


def _run(binary, *args):
    proc = subprocess.run([str(binary), *args], capture_output=True, text=True, timeout=600)
    checked, failures = map(int, proc.stdout.split())
    return proc.returncode, checked, failures


def test_division_by_127_is_ieee_on_its_whole_domain(checker):
    rc, checked, failures = _run(checker, "div127")
    assert checked > 3_000_000_000 and failures == 0 and rc == 0


def test_two_part_division_by_127_is_ieee_on_its_whole_domain(checker):
    """div_by_127 (q = RN(a * R + RN(a * L)), the dequantize's division) for
    every float with 2^-100 <= |a| < 2^121 and both zeros."""
    rc, checked, failures = _run(checker, "div127split")
    assert checked > 3_000_000_000 and failures == 0 and rc == 0


def test_division_by_random_divisors_is_ieee(checker):
    rc, checked, failures = _run(checker, "divrandom", "48")
    assert checked == 48 * 2 * (1 << 23) and failures == 0 and rc == 0


def test_refit_division_is_ieee_at_the_edges_of_its_fast_domain(checker):
    """The quant-only refit divides w / s by the reciprocal of the smoothing
    value when s is in [2^-20, 2^20] and w is 0 or in [2^-100, 2^100]
    (csrc/boundary.hip): divisors at the domain's edges, with power-of-two and
    all-ones significands, against every dividend significand at its edges."""
    rc, checked, failures = _run(checker, "refit")
    assert checked == 25 * (2 * 2 * (1 << 23) + 2) and failures == 0 and rc == 0


def test_rounding_matches_lround_for_every_float_up_to_127(checker):
    rc, checked, failures = _run(checker, "round")
    assert checked > 2_000_000_000 and failures == 0 and rc == 0


def test_lifted_codes_match_lround_wherever_the_margin_admits_them(checker):
    """The encoder's lifted code (floor of code_lift's fma, lifted_code in
    codec_math.h) against clamp(lround(m / scale * 127)) in IEEE fp32: every float m of one
    scale, random scales over [2^-90, 2^90] with random m, and m within 200 ulps
    of every tie point.  With the margin lowered to 2^-20 this check fails
    (about 1.3e7 mismatches), so the margin is what makes it pass."""
    rc, checked, failures = _run(checker, "lift")
    assert checked > 3_000_000_000 and failures == 0 and rc == 0


def test_lifted_codes_match_the_refit_rounding_wherever_the_margin_admits_them(checker):
    """The same sweep against the window-boundary re-encode's own rounding,
    trunc(RN(q +- 0.5)) clamped to +-127 (window_boundary.cpp:336-345), which
    the power refit and encoded_requantize now take from the lifted code."""
    rc, checked, failures = _run(checker, "lift_refit")
    assert checked > 3_000_000_000 and failures == 0 and rc == 0


def test_bf16_direct_lift_matches_lround_wherever_its_margin_admits_it(checker):
    """The bf16 pool encoder's codes formed from the kept product
    q0 = RN(r * RN(1/s)) (wide_code_lift in codec_math.h) against
    clamp(lround(RN(RN(RN(r/s) / scale) * 127))) in IEEE fp32, and the exact
    path's recovery of r (bit for bit) and of m = RN(r/s) from q0: every bf16 r
    of 16,384 random (s, scale) pairs over the fast domains.  With the margin
    lowered to 2^-15 (34,537 mismatches), the offset to 0.5 (6,280), or the
    recovery's rounding to bf16 left out (1.2e8), this check fails, so those
    are what make it pass."""
    rc, checked, failures = _run(checker, "wide_lift")
    assert checked > 400_000_000 and failures == 0 and rc == 0


def test_xcd_contiguous_order_is_a_bijection(checker):
    """The streaming kernels' workgroup -> tile order (csrc/work_order.h) visits
    every tile exactly once for every grid size up to 4,096 and the bench's."""
    rc, checked, failures = _run(checker, "order")
    assert checked == 4096 + 7 and failures == 0 and rc == 0
