"""CPU tests of the encoder: the oracle restatement (oracle/ckks_encode.py)
pinned against the mathematics it implements, and the library's host half
(chd_encode_coefficients, no device) against the oracle, bit-exact.

Pins: the special IFFT inverts the canonical embedding
z_j = sum_k a_k zeta_{4s}^(k 5^j) evaluated directly (O(s^2)); the Galois
automorphism X -> X^(5^r) of an encoded integer polynomial rotates the
slots left by r (the rotation the reference's HRot / Hoist maps assume);
truncation and residues agree with Python's exact integer conversion;
decode's CRT recovers signed integer coefficients.
"""
import math

import numpy as np
import pytest

import ckks_encode as E
from gpu_util import config4


def _msg(seed, n, lo=-1.0, hi=1.0):
    r = np.random.default_rng(seed)
    return r.uniform(lo, hi, n) + 1j * r.uniform(lo, hi, n)


@pytest.mark.parametrize("s,m", [(256, 4096), (1024, 1 << 17)])
def test_special_ifft_inverts_canonical_embedding(s, m):
    z = _msg(1, s)
    re, im = z.real.copy(), z.imag.copy()
    E.special_ifft(re, im, m)
    a = re + 1j * im
    g = E.galois_factors(s, 4 * s)
    zeta = np.exp(2j * np.pi * (np.outer(g, np.arange(s)) % (4 * s)) / (4 * s))
    assert np.max(np.abs(zeta @ a - z)) < 1e-12


def test_special_fft_inverts_special_ifft():
    z = _msg(2, 1 << 15)
    re, im = z.real.copy(), z.imag.copy()
    E.special_ifft(re, im, 1 << 17)
    E.special_fft(re, im, 1 << 17)
    assert np.max(np.abs(re + 1j * im - z)) < 1e-12


def test_galois_automorphism_rotates_slots_left():
    log_n = 10
    n = 1 << log_n
    s = n // 2
    scale = 2.0 ** 40
    z = _msg(3, s)
    re, im = z.real.copy(), z.imag.copy()
    E.special_ifft(re, im, 2 * n)
    coef = [0] * n
    for k in range(s):
        coef[k] = int(math.trunc(re[k] * scale))
        coef[k + s] = int(math.trunc(im[k] * scale))
    for r in (1, 5, 100):
        g = pow(5, r, 2 * n)
        rot = [0] * n
        for i, c in enumerate(coef):
            j = i * g % (2 * n)
            if j < n:
                rot[j] += c
            else:
                rot[j - n] -= c
        rr = np.array([rot[k] / scale for k in range(s)])
        ri = np.array([rot[k + s] / scale for k in range(s)])
        E.special_fft(rr, ri, 2 * n)
        assert np.max(np.abs(rr + 1j * ri - np.roll(z, -r))) < 1e-6


def test_trunc_mod_matches_exact_integer_conversion():
    p = 1073479681
    vals = np.array([0.0, -0.0, 0.5, -0.5, 1.9999, -1.9999, p - 0.5, -p + 0.25,
                     2.0 ** 62 + 4096, -(2.0 ** 62), 2.0 ** 63, -(2.0 ** 63),
                     1e30, -1e30, 3.3e300, -7.1e200, 1e-300, -1e-300])
    got = E.trunc_mod(vals, p)
    want = [int(v) % p for v in vals.tolist()]
    assert got.tolist() == want


def test_tommath_get_double_below_one_digit_is_exact_rounding():
    r = np.random.default_rng(4)
    for bits in (1, 30, 52, 53, 59, 60):
        for _ in range(50):
            v = int(r.integers(0, 1 << 62)) >> (62 - bits)
            assert E.tommath_get_double(v) == float(v)
            assert E.tommath_get_double(-v) == -float(v)
    # two digits: hi * 2^60 + lo, hi exact in a double
    assert E.tommath_get_double((3 << 60) + 5) == float(3 << 60)


def test_decode_crt_recovers_signed_coefficients():
    log_n = 10
    n = 1 << log_n
    primes = [1073479681, 1073217537, 1072693249]  # 30-bit, 1 mod 2^11
    scale = 2.0 ** 30
    r = np.random.default_rng(5)
    coef = [int(v) for v in r.integers(-(1 << 45), 1 << 45, n)]
    scaled = np.zeros((len(primes), n), np.uint32)
    Q = math.prod(primes)
    for i, q in enumerate(primes):
        inv = pow(Q // q, -1, q)
        scaled[i] = [c % q * inv % q for c in coef]
    re, im = E.decode_values(scaled, primes, log_n, n // 2, scale)
    wr = np.array(coef[:n // 2], np.float64) / scale
    wi = np.array(coef[n // 2:], np.float64) / scale
    E.special_fft(wr, wi, 2 * n)
    assert np.array_equal(re, wr) and np.array_equal(im, wi)


def test_encode_constant_is_montgomery_of_truncated_value():
    primes = [1073479681, 2147352577]
    for number, scale in ((0.7, 2.0 ** 30), (-3.25, 2.0 ** 40),
                          (1.5, 2.0 ** 80)):
        cx = E.encode_constant(number, primes, scale)
        v = int(number * scale)
        for c, p in zip(cx.tolist(), primes):
            assert c * pow(1 << 32, -1, p) % p == v % p


# ------------------------------------ library host half against the oracle --
@pytest.fixture(scope="module")
def param():
    import cheddar_amd
    main, aux, levels = config4()
    return cheddar_amd.Param(main, aux, levels)


@pytest.mark.parametrize("level,num_aux,length,scale", [
    (23, 0, 1 << 15, 2.0 ** 30),
    (0, 0, 3, 2.0 ** 30),
    (19, 8, 1 << 15, 2.0 ** 30),
    (5, 8, 100, 2.0 ** 75),      # values beyond 2^63
    (11, 0, 1, 2.0 ** 40),
    (7, 0, 1000, 2.0 ** 52),
])
def test_host_residues_match_oracle(param, level, num_aux, length, scale):
    msg = _msg(100 + level + length, length, -4.0, 4.0)
    got, slots = param.encode_coefficients(level, num_aux, scale, msg)
    primes = param.main[:param.num_q(level)] + param.aux[:num_aux]
    want, wslots = E.coefficient_residues(msg.real, msg.imag, primes, 16,
                                          scale)
    assert slots == wslots
    assert np.array_equal(got, want)


def test_host_residues_reject_invalid(param):
    import cheddar_amd
    with pytest.raises(cheddar_amd.ChdError):
        param.encode_coefficients(23, 3, 2.0 ** 30, _msg(1, 4))  # aux not alpha
    with pytest.raises(cheddar_amd.ChdError, match="finite"):
        param.encode_coefficients(3, 0, 2.0 ** 30, np.array([np.inf + 0j]))
