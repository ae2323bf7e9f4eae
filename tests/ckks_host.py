"""Host-side CKKS helpers for semantic tests: a known ternary secret, key
generation with the reference's gadget (UserInterface.cu:366-458: group g of
evk.bx carries P * s' on its own limbs), encryption of integer polynomials
and decryption by CRT. Residues are NTT-domain Montgomery form
(NTT(x * R)), the form the reference keeps ciphertexts and keys in.

Test infrastructure only.
"""
import numpy as np

import _orc

R = 1 << 32


def crt_centre(residues, primes):
    """residues: [len(primes)][N] -> list of centred Python ints."""
    Q = 1
    for p in primes:
        Q *= p
    n = residues.shape[1]
    out = [0] * n
    for i, p in enumerate(primes):
        qh = Q // p
        f = qh * pow(qh % p, -1, p)
        col = residues[i].tolist()
        for c in range(n):
            out[c] += col[c] * f
    res = []
    for v in out:
        v %= Q
        if v > Q // 2:
            v -= Q
        res.append(v)
    return res


def to_ntt_mont(coeffs, primes, log_n):
    """integer coefficient vector (Python ints or int64) -> NTT(x R) limbs"""
    coeffs = [int(v) for v in coeffs]
    limbs = np.zeros((len(primes), 1 << log_n), np.uint32)
    for i, p in enumerate(primes):
        limbs[i] = np.array([v % p for v in coeffs], dtype=np.uint32)
    return _orc.ntt_batch(limbs.reshape(-1), log_n, primes, mont=1).reshape(
        len(primes), -1)


def from_ntt_mont(limbs, primes, log_n):
    """NTT-domain Montgomery limbs -> centred integer coefficients via CRT"""
    coef = _orc.intt_batch(np.ascontiguousarray(limbs).reshape(-1), log_n,
                           primes, mont=1).reshape(len(primes), -1)
    return crt_centre(coef, primes)


def mont_mul_vec(a, b, q):
    ri = pow(R, -1, q)
    return (a.astype(np.uint64) * b % q * ri % q).astype(np.uint32)


class Keys:
    """secret s (ternary, fixed seed) and NTT-Montgomery forms per prime"""

    def __init__(self, log_n, q_primes, p_primes, seed=1):
        self.log_n = log_n
        self.n = 1 << log_n
        self.q = list(q_primes)
        self.p = list(p_primes)
        self.rng = np.random.default_rng(seed)
        self.s = self.rng.integers(-1, 2, self.n).astype(np.int64)
        self.all_primes = self.q + self.p
        self.s_ntt = to_ntt_mont(self.s, self.all_primes, log_n)

    def ntt_of(self, coeffs, primes):
        return to_ntt_mont(coeffs, primes, self.log_n)

    def _mul(self, a, b, primes):
        out = np.zeros_like(a)
        for i, p in enumerate(primes):
            out[i] = mont_mul_vec(a[i], b[i], p)
        return out

    def _add(self, a, b, primes):
        out = np.zeros_like(a)
        for i, p in enumerate(primes):
            out[i] = ((a[i].astype(np.uint64) + b[i]) % p).astype(np.uint32)
        return out

    def _neg(self, a, primes):
        out = np.zeros_like(a)
        for i, p in enumerate(primes):
            out[i] = ((p - a[i].astype(np.uint64)) % p).astype(np.uint32)
        return out

    def uniform(self, primes):
        return np.stack([self.rng.integers(0, p, self.n, dtype=np.uint64)
                         .astype(np.uint32) for p in primes])

    def small(self, bound=4):
        return self.rng.integers(-bound, bound + 1, self.n)

    def encrypt(self, m, L):
        """(b, a) over q_0..q_{L-1} with b = -a s + m + e"""
        primes = self.q[:L]
        a = self.uniform(primes)
        m_e = (np.asarray(m, dtype=object) + self.small()).tolist()
        b = self._add(self._neg(self._mul(a, self.s_ntt[:L], primes), primes),
                      self.ntt_of(m_e, primes), primes)
        return b, a

    def decrypt(self, b, a, L):
        primes = self.q[:L]
        v = self._add(b, self._mul(a, self.s_ntt[:L], primes), primes)
        return from_ntt_mont(v, primes, self.log_n)

    def switch_key(self, s_new, max_q, s_enc=None):
        """evk for target secret s_new (coefficients) encrypted under s_enc
        (default s), beta groups of (max_q + alpha) limbs;
        bx_g = -a_g s_enc + e_g + P s_new on group g (UserInterface.cu:366)."""
        alpha = len(self.p)
        primes = self.q[:max_q] + self.p
        beta = (max_q + alpha - 1) // alpha
        if s_enc is None:
            s_cur = np.concatenate([self.s_ntt[:max_q],
                                    self.s_ntt[len(self.q):]])
        else:
            s_cur = self.ntt_of(s_enc, primes)
        t = self.ntt_of(s_new, primes)
        P = 1
        for p in self.p:
            P *= p
        kb, ka = [], []
        for g in range(beta):
            a = self.uniform(primes)
            b = self._add(self._neg(self._mul(a, s_cur, primes), primes),
                          self.ntt_of(self.small(), primes), primes)
            for i in range(g * alpha, min((g + 1) * alpha, max_q)):
                q = primes[i]
                pm = (P % q) * R % q  # ToMont(P mod q)
                add = mont_mul_vec(t[i], np.full(self.n, pm, np.uint32), q)
                b[i] = ((b[i].astype(np.uint64) + add) % q).astype(np.uint32)
            kb.append(b)
            ka.append(a)
        return np.stack(kb), np.stack(ka)

    def mult_key(self, max_q):
        s2 = negacyclic_mul(self.s, self.s)
        return self.switch_key(s2, max_q)

    def rot_key(self, galois, max_q):
        """HRot key-switches first and permutes after (Context.cpp:776-791),
        so the key encrypts s under s(X^(g^-1)) (UserInterface.cu:279-306)"""
        g_inv = pow(galois, -1, 2 * self.n)
        return self.switch_key(self.s, max_q,
                               s_enc=automorphism(self.s, g_inv))


def negacyclic_mul(a, b):
    """schoolbook product mod X^N + 1 with Python-int exactness"""
    a = np.asarray(a, dtype=object)
    b = np.asarray(b, dtype=object)
    n = len(a)
    full = np.convolve(a, b)
    out = full[:n].copy()
    out[: n - 1] -= full[n:]
    return out


def automorphism(a, g):
    """coefficients of a(X^g) mod X^N + 1"""
    n = len(a)
    out = np.zeros(n, dtype=object)
    for j, v in enumerate(np.asarray(a, dtype=object)):
        e = (j * g) % (2 * n)
        if e >= n:
            out[e - n] -= v
        else:
            out[e] += v
    return out
