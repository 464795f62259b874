"""Device arithmetic checked on the host (no GPU): R1's certified bf16 rounding, built for the host
from the same source the kernels use (csrc/router_dev.h via csrc/hostcheck/), against the oracle's
midpoint rule and exact rounding."""
import ctypes
from pathlib import Path

import numpy as np
import pytest

from oracle import moe_oracle as O

LIB = Path(__file__).resolve().parents[1] / "qwen3.6-35b-a3b_amd" / "libmoe_hostcheck.so"


@pytest.fixture(scope="module")
def certify():
    if not LIB.exists():
        pytest.fail(f"{LIB} is not built: run __graft_entry__.build() first")
    lib = ctypes.CDLL(str(LIB))
    f = lib.moe_hostcheck_round_bf16
    f.argtypes = [ctypes.c_double, ctypes.c_double, ctypes.POINTER(ctypes.c_uint32)]
    f.restype = ctypes.c_int

    def call(s, bound):
        b = ctypes.c_uint32(0xDEAD)
        ok = f(float(s), float(bound), ctypes.byref(b))
        return bool(ok), b.value
    return call


def _bf16_bits(v: float) -> int:
    return int(np.array([v], dtype=np.float32).view(np.uint32)[0] >> 16)


def test_lower_midpoint_just_above_a_power_of_two(certify):
    """s = 2^e + f q (q = 2^(e-7)): the midpoint below 2^e is at (f + 1/4) q, nearer than the one
    at (1/2 - f) q when f < 1/8, so a bound between the two must not certify."""
    for e in (-20, -1, 0, 5, 40):
        q = 2.0 ** (e - 7)
        for f in (0.0, 0.03125, 0.1):
            s = 2.0 ** e + f * q
            lower, upper = (f + 0.25) * q, (0.5 - f) * q
            bound = 0.5 * (lower + upper)
            assert certify(s, bound)[0] is False, (e, f)
            assert certify(-s, bound)[0] is False, (e, f)
            ok, bits = certify(s, 0.9 * lower)
            assert ok and bits == _bf16_bits(2.0 ** e)


def test_subnormal_range_has_one_quantum(certify):
    """Below 2^-126 (and across it) the bf16 quantum stays 2^-133: no lower midpoint."""
    s = 2.0 ** -126
    ok, bits = certify(s, 0.4 * 2.0 ** -133)
    assert ok and bits == 0x0080


def test_agrees_with_the_oracle_midpoint_rule_and_exact_rounding(certify):
    """certified <=> the oracle's midpoint distance exceeds the bound; certified bits = the exact
    bf16 rounding of s (round_f64_to_bf16), over values near powers of two, midpoints and
    random magnitudes."""
    rng = np.random.default_rng(11)
    vals = []
    for e in rng.integers(-60, 60, 300):
        q = 2.0 ** (int(e) - 7)
        vals += [2.0 ** int(e) + rng.uniform(0, 0.3) * q, 2.0 ** int(e) - rng.uniform(0, 0.3) * q / 2,
                 2.0 ** int(e) + (rng.integers(0, 128) + 0.5) * q * (1 + rng.uniform(-1e-3, 1e-3))]
    vals += list(rng.standard_normal(300) * 10.0 ** rng.uniform(-8, 8, 300))
    s = np.array(vals) * np.where(rng.random(len(vals)) < 0.5, -1.0, 1.0)
    dist = O.midpoint_distance(s)
    ref_bits = O.round_f64_to_bf16(s).astype(np.float32).view(np.uint32) >> 16
    for k, v in enumerate(s):
        for bound in (0.0, 0.999 * dist[k], 1.001 * dist[k]):
            ok, bits = certify(v, bound)
            assert ok == (dist[k] > bound), (v, bound, dist[k])
            if ok:
                assert bits == int(ref_bits[k]), (v, hex(bits), hex(int(ref_bits[k])))
