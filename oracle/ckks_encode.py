"""CPU restatement of the CKKS encoder (src/core/Encode.cpp) -- test
infrastructure only: the checker for the encoder entry points, never called
by the product.

Every floating-point step is one IEEE double operation in the reference's
order, written with explicit real arithmetic so no product and sum can fuse:
a complex product (a + bi)(c + di) is (ac - bd) + (ad + bc)i, each product
rounded, as the reference's host build computes it (-O3, no FMA target).
Twiddles come from math.cos / math.sin (the C library's, as std::polar uses).
Integer steps use Python integers (exact).

Functions and the reference lines they follow:
  twiddles            Encode.cpp:10-21   e^(2 pi i k / M), M = 2N
  special_ifft        Encode.cpp:84-109  (+ BitReverseVector, CommonUtils.h)
  special_fft         Encode.cpp:111-133
  coefficient_residues Encode.cpp:23-43, 135-190 (pad, IFFT, scale,
                      BigInt(double) truncation, non-negative mod)
  decode_values       Encode.cpp:45-82, 192-246 (iCRT, NormalizeMod,
                      mp_get_double of libtommath, / scale, SpecialFFT)
  encode_constant     Encode.cpp:248-273
"""
import math

import numpy as np


def galois_factors(count, m):
    """5^j mod M for j < count (Parameter.cu's galois factor table)."""
    out = np.empty(count, np.int64)
    g = 1
    for j in range(count):
        out[j] = g
        g = g * 5 % m
    return out


def twiddles(m):
    """(re, im) of std::polar(1.0, 2.0 * M_PI * k / M): the angle is
    ((2.0 * pi) * k) / M, each step rounded."""
    re = np.empty(m, np.float64)
    im = np.empty(m, np.float64)
    two_pi = 2.0 * math.pi
    for k in range(m):
        t = two_pi * k / m
        re[k] = math.cos(t)
        im[k] = math.sin(t)
    return re, im


_TW_CACHE = {}


def _tw(m):
    if m not in _TW_CACHE:
        _TW_CACHE[m] = twiddles(m)
    return _TW_CACHE[m]


def _bitrev_perm(n):
    bits = n.bit_length() - 1
    idx = np.arange(n)
    r = np.zeros(n, np.int64)
    for b in range(bits):
        r |= ((idx >> b) & 1) << (bits - 1 - b)
    return r


def special_ifft(re, im, m):
    """In place on float64 arrays re, im (length = slots, a power of two)."""
    s = re.size
    assert s & (s - 1) == 0
    twr, twi = _tw(m)
    gal = galois_factors(max(s // 2, 1), m)
    stride = s // 2
    while stride >= 1:
        st8 = stride << 3
        gap = m // st8
        idx = (st8 - gal[:stride] % st8) * gap
        wr, wi = twr[idx], twi[idx]
        vr = re.reshape(-1, 2, stride)
        vi = im.reshape(-1, 2, stride)
        ur, ui = vr[:, 0, :].copy(), vi[:, 0, :].copy()
        lr, li = vr[:, 1, :].copy(), vi[:, 1, :].copy()
        xr, xi = ur + lr, ui + li
        yr, yi = ur - lr, ui - li
        vr[:, 0, :] = xr
        vi[:, 0, :] = xi
        vr[:, 1, :] = yr * wr - yi * wi
        vi[:, 1, :] = yr * wi + yi * wr
        stride //= 2
    p = _bitrev_perm(s)
    re[:] = re[p] / s
    im[:] = im[p] / s


def special_fft(re, im, m):
    """In place; the inverse map of special_ifft up to rounding."""
    s = re.size
    assert s & (s - 1) == 0
    twr, twi = _tw(m)
    gal = galois_factors(max(s // 2, 1), m)
    p = _bitrev_perm(s)
    re[:] = re[p]
    im[:] = im[p]
    stride = 1
    while stride < s:
        st8 = stride << 3
        gap = m // st8
        idx = (gal[:stride] % st8) * gap
        wr, wi = twr[idx], twi[idx]
        vr = re.reshape(-1, 2, stride)
        vi = im.reshape(-1, 2, stride)
        xr, xi = vr[:, 0, :].copy(), vi[:, 0, :].copy()
        lr, li = vr[:, 1, :], vi[:, 1, :]
        yr = lr * wr - li * wi
        yi = lr * wi + li * wr
        vr[:, 0, :] = xr + yr
        vi[:, 0, :] = xi + yi
        vr[:, 1, :] = xr - yr
        vi[:, 1, :] = xi - yi
        stride *= 2


def trunc_mod(values, p):
    """BigInt(double) (truncation toward zero) then BigInt::Mod (result in
    [0, p)) for a float64 array; exact for every finite double."""
    v = np.asarray(values, np.float64)
    assert np.all(np.isfinite(v))
    t = np.trunc(v)
    out = np.empty(v.shape, np.uint32)
    small = np.abs(t) < 2.0 ** 63
    out[small] = (t[small].astype(np.int64) % p).astype(np.uint32)
    for k in np.flatnonzero(~small):
        out.flat[k] = int(t.flat[k]) % p
    return out


def padded_slots(length):
    s = 1
    while s < length:
        s <<= 1
    return s


def coefficient_residues(msg_re, msg_im, primes, log_n, scale):
    """Message -> [len(primes)][N] coefficient residues (before the NTT)."""
    n = 1 << log_n
    m = 2 * n
    half = n // 2
    slots = padded_slots(len(msg_re))
    assert slots <= half
    re = np.zeros(slots, np.float64)
    im = np.zeros(slots, np.float64)
    re[:len(msg_re)] = msg_re
    im[:len(msg_im)] = msg_im
    special_ifft(re, im, m)
    gap = half // slots
    vr, vi = re * scale, im * scale
    mx = np.zeros((len(primes), n), np.uint32)
    pos = np.arange(slots) * gap
    for j, p in enumerate(primes):
        mx[j, pos] = trunc_mod(vr, p)
        mx[j, pos + half] = trunc_mod(vi, p)
    return mx, slots


def encode_constant(number, primes, scale):
    """trunc(number * scale) mod p, then ToMontgomery (x 2^32 mod p)."""
    v = int(math.trunc(number * scale))
    return np.array([(v % p) * (1 << 32) % p for p in primes], np.uint32)


def tommath_get_double(v):
    """libtommath's mp_get_double: 60-bit digits from the most significant,
    d = d * 2^60 + (double)digit, each step rounded; then the sign."""
    neg = v < 0
    mag = -v if neg else v
    digits = []
    while mag:
        digits.append(mag & ((1 << 60) - 1))
        mag >>= 60
    d = 0.0
    for dg in reversed(digits):
        d = d * 2.0 ** 60 + float(dg)
    return -d if neg else d


def icrt_constants(primes, n):
    """(N prod_{k != i} q_k)^-1 mod q_i, not in Montgomery form."""
    out = []
    for i, q in enumerate(primes):
        prod = 1
        for j, qj in enumerate(primes):
            if j != i:
                prod = prod * qj % q
        prod = prod * n % q
        out.append(pow(prod, -1, q))
    return out


def decode_values(scaled_residues, primes, log_n, num_slots, scale):
    """scaled_residues: INTTAndMultConst's output with icrt_constants, i.e.
    coefficient_i * (prod_{k != i} q_k)^-1 mod q_i, [len(primes)][N].
    Returns (re, im) float64 arrays of num_slots decoded values."""
    n = 1 << log_n
    half = n // 2
    gap = half // num_slots
    Q = 1
    for q in primes:
        Q *= q
    half_q = Q // 2
    qhat = [Q // q for q in primes]
    cols = [r.tolist() for r in scaled_residues]

    def value(idx):
        acc = 0
        for j in range(len(primes)):
            acc += cols[j][idx] * qhat[j]
        acc %= Q
        if acc > half_q:
            acc -= Q
        return tommath_get_double(acc)

    re = np.array([value(i * gap) / scale for i in range(num_slots)],
                  np.float64)
    im = np.array([value(i * gap + half) / scale for i in range(num_slots)],
                  np.float64)
    special_fft(re, im, 2 * n)
    return re, im
