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
    limbs = np.zeros((len(primes), 1 << log_n), np.uint32)
    c = np.asarray(coeffs)
    if c.dtype.kind in "iu":
        c = c.astype(np.int64)
        for i, p in enumerate(primes):
            limbs[i] = np.mod(c, p).astype(np.uint32)
    else:
        coeffs = [int(v) for v in coeffs]
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

    def uniform(self, primes, rng=None):
        rng = self.rng if rng is None else rng
        out = np.empty((len(primes), self.n), np.uint32)
        for i, p in enumerate(primes):
            out[i] = rng.integers(0, p, self.n, dtype=np.uint64)
        return out

    def small(self, bound=4, rng=None):
        rng = self.rng if rng is None else rng
        return rng.integers(-bound, bound + 1, self.n)

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

    def switch_key(self, s_new, max_q, s_enc=None, rng=None, s_new_ntt=None):
        """evk for target secret s_new (coefficients) encrypted under s_enc
        (default s), beta groups of (max_q + alpha) limbs;
        bx_g = -a_g s_enc + e_g + P s_new on group g (UserInterface.cu:366).
        Vectorised over all limbs of a group (one modulus per row); rng
        (default: the secret's generator) draws a and the errors.
        s_new_ntt: s_new already in NTT-Montgomery form over those primes
        (then s_new is not read)."""
        alpha = len(self.p)
        primes = self.q[:max_q] + self.p
        beta = (max_q + alpha - 1) // alpha
        total = len(primes)
        own = np.concatenate([self.s_ntt[:max_q], self.s_ntt[len(self.q):]])
        s_cur = own if s_enc is None else self.ntt_of(s_enc, primes)
        t = (s_new_ntt if s_new_ntt is not None else
             own if s_new is self.s else self.ntt_of(s_new, primes))
        pc = np.array(primes, np.uint64)[:, None]
        r_inv = np.array([pow(R, -1, p) for p in primes], np.uint64)[:, None]
        P = 1
        for p in self.p:
            P *= p
        p_mod = np.array([P % p for p in primes], np.uint64)[:, None]
        # errors of every group in one batched NTT
        e = np.zeros((beta, total, self.n), np.uint32)
        for g in range(beta):
            c = self.small(rng=rng).astype(np.int64)
            e[g] = np.mod(c[None, :], pc.astype(np.int64)).astype(np.uint32)
        e = _orc.ntt_batch(e.reshape(-1), self.log_n, primes * beta,
                           mont=1).reshape(beta, total, self.n)
        s64 = s_cur.astype(np.uint64)
        pt = t.astype(np.uint64) * p_mod % pc  # MontMul(t, ToMont(P mod q))
        kb, ka = [], []
        for g in range(beta):
            a = self.uniform(primes, rng)
            a_s = (a.astype(np.uint64) * s64 % pc) * r_inv % pc
            b = (e[g].astype(np.uint64) + pc - a_s) % pc
            lo, hi = g * alpha, min((g + 1) * alpha, max_q)
            b[lo:hi] = (b[lo:hi] + pt[lo:hi]) % pc[lo:hi]
            kb.append(b.astype(np.uint32))
            ka.append(a)
        return np.stack(kb), np.stack(ka)

    def mult_key(self, max_q):
        s2 = negacyclic_mul(self.s, self.s)
        return self.switch_key(s2, max_q)

    def mult_key_ntt(self, max_q, rng=None):
        """the same key with s^2 formed pointwise in the NTT domain
        (MontMul of s's NTT-Montgomery limbs with themselves is the NTT of
        the negacyclic square): no O(N^2) product, for N = 2^16"""
        own = np.concatenate([self.s_ntt[:max_q], self.s_ntt[len(self.q):]])
        primes = self.q[:max_q] + self.p
        s2 = np.stack([mont_mul_vec(own[i], own[i], p)
                       for i, p in enumerate(primes)])
        return self.switch_key(None, max_q, rng=rng, s_new_ntt=s2)

    def rot_key(self, galois, max_q, rng=None):
        """HRot key-switches first and permutes after (Context.cpp:776-791),
        so the key encrypts s under s(X^(g^-1)) (UserInterface.cu:279-306)"""
        g_inv = pow(galois, -1, 2 * self.n)
        return self.switch_key(self.s, max_q,
                               s_enc=automorphism(self.s, g_inv), rng=rng)


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
    """coefficients of a(X^g) mod X^N + 1 (g odd: j -> j g mod N is a
    permutation, so every output coefficient receives exactly one term)"""
    a = np.asarray(a)
    if a.dtype.kind in "iu":
        a = a.astype(np.int64)
    n = len(a)
    assert g % 2 == 1
    e = (np.arange(n, dtype=np.int64) * g) % (2 * n)
    neg = e >= n
    out = np.zeros(n, dtype=np.int64 if a.dtype.kind == "i" else object)
    out[np.where(neg, e - n, e)] = np.where(neg, -a, a)
    return out
