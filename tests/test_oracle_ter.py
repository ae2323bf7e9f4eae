"""CPU pins of the oracle's terminal-prime pieces (orc_mod_up_ex,
orc_mod_down_ex, orc_paccum_ex) and of the compositions in tests/ks_ref.py:

- ModDown with the BitPacker restore against its closed form: for input X,
  the output V (over the destination primes) and the BConv term E satisfy
  D V + E = X R exactly, D the product of the dropped primes, R of the
  restored ones, E = sum_i c_i D/q_i with c_i the centred residues of X R
  (D/q_i)^-1 (ModSwitch.cu:258-411, NTT.cu:456-601);
- without restore, orc_mod_down_ex equals the pinned orc_mod_down;
- ModUp with a prime offset: the fast base conversion invariants per group;
- with no terminal primes the compositions equal the pinned orc_hmult /
  orc_mult_key / orc_hrot;
- with terminal primes, semantic decryption under a known secret through
  HMult + rescales that drop main primes and restore terminal ones and vice
  versa, and HRot at a level with a prime offset.
"""
import math

import numpy as np
import pytest

import _orc
import ckks_host as ck
from chd_primes import ntt_primes
from ks_ref import Chain

Q30 = ntt_primes(30, 16)
Q31 = ntt_primes(31, 8)
Q25 = ntt_primes(25, 8)


def rng(seed):
    return np.random.default_rng(seed)


def _rand_poly(r, n, bits):
    hi = r.integers(-(1 << (bits - 40)), 1 << (bits - 40), n)
    lo = r.integers(0, 1 << 40, n)
    return [(int(h) << 40) + int(l) for h, l in zip(hi, lo)]


def _centred_residue(v, q):
    v %= q
    return v - q if v > q // 2 else v


@pytest.mark.parametrize("case", ["ter_drop_main_restore",
                                  "main_drop_ter_restore", "merged_with_aux",
                                  "plain_rescale"])
def test_mod_down_ex_closed_form(case):
    log_n = 8
    n = 1 << log_n
    a, b, c, d = Q30[:4]
    t0, t1, t2 = Q25[:3]
    p0, p1 = Q31[:2]
    if case == "ter_drop_main_restore":      # (main 1, ter 3) -> (2, 1)
        src_p = [t2, t1, t0, a]
        drop = [0, 1]
        dst_p = [t0, a, b]
    elif case == "main_drop_ter_restore":    # (3, 1) -> (1, 3)
        src_p = [t0, a, b, c]
        drop = [2, 3]
        dst_p = [t2, t1, t0, a]
    elif case == "merged_with_aux":          # (3, 1) + P -> (1, 2)
        src_p = [t0, a, b, c, p0, p1]
        drop = [2, 3, 4, 5]
        dst_p = [t1, t0, a]
    else:                                    # (4, 0) -> (3, 0)
        src_p = [a, b, c, d]
        drop = [3]
        dst_p = [a, b, c]
    D = math.prod(src_p[i] for i in drop)
    Rr = math.prod(p for p in dst_p if p not in src_p)
    Qs = math.prod(src_p)
    r = rng(hash(case) % 1000)
    X = [int(v) for v in r.integers(-(1 << 62), 1 << 62, n)]
    X = [v * (Qs >> 66) for v in X]                  # |X| < Qs / 16
    src = ck.to_ntt_mont(X, src_p, log_n)
    keep = {p: i for i, p in enumerate(src_p) if i not in drop}
    dst_src = [keep.get(p, -1) for p in dst_p]
    out = _orc.mod_down_ex(src, src_p, drop, dst_p, dst_src, log_n)
    V = ck.from_ntt_mont(out, dst_p, log_n)
    for j in (0, 1, 77, n - 1):
        E = 0
        for i in drop:
            q = src_p[i]
            qh = D // q
            E += _centred_residue(X[j] * Rr * pow(qh % q, -1, q), q) * qh
        assert D * V[j] + E == X[j] * Rr, (case, j)


def test_mod_down_ex_without_restore_equals_mod_down():
    log_n = 8
    primes = Q30[:5] + Q31[:3]
    r = rng(3)
    src = np.stack([r.integers(0, p, 1 << log_n, dtype=np.uint64)
                    .astype(np.uint32) for p in primes])
    for keep in (5, 4):
        want = _orc.mod_down(src, primes, keep, log_n)
        drop = list(range(keep, len(primes)))
        got = _orc.mod_down_ex(src, primes, drop, primes[:keep],
                               list(range(keep)), log_n)
        assert np.array_equal(got, want)


@pytest.mark.parametrize("offset,alpha", [(1, 3), (2, 3), (3, 2)])
def test_mod_up_ex_invariants(offset, alpha):
    log_n = 8
    n = 1 << log_n
    qp, pp = Q30[:5], Q31[:alpha]
    L = len(qp)
    primes = qp + pp
    r = rng(10 + offset)
    x = np.stack([r.integers(0, q, n, dtype=np.uint64).astype(np.uint32)
                  for q in qp])
    out = _orc.mod_up_ex(x, qp, pp, offset, log_n)
    beta = (L + offset + alpha - 1) // alpha
    assert out.shape[0] == beta
    coef = _orc.intt_batch(x.reshape(-1), log_n, qp, 1).reshape(L, -1)
    seen = 0
    for g in range(beta):
        e_abs = min((g + 1) * alpha, L + offset)
        if e_abs <= offset:
            assert not out[g].any()
            continue
        s, e = max(0, g * alpha - offset), e_abs - offset
        seen += e - s
        grp = qp[s:e]
        Qg = math.prod(grp)
        assert np.array_equal(out[g, s:e], x[s:e])
        oc = _orc.intt_batch(out[g].reshape(-1), log_n, primes, 1).reshape(
            L + alpha, -1)
        for c in (0, 5, n - 1):
            X = 0
            for i, q in enumerate(grp):
                qh = Qg // q
                X += _centred_residue(int(coef[s + i, c]) * pow(qh % q, -1, q),
                                      q) * qh
            assert abs(X) <= len(grp) * Qg // 2
            for j, p in enumerate(primes):
                assert int(oc[j, c]) == X % p
    assert seen == L


def test_compositions_without_terminal_primes_equal_fixed_oracle():
    log_n = 8
    n = 1 << log_n
    main, aux = Q30[:6], Q31[:3]
    chain = Chain(main, [], aux, [(i, 0) for i in range(1, 7)], log_n)
    r = rng(5)
    L, level = 5, 4
    q = main[:L]

    def uni(primes):
        return np.stack([r.integers(0, p, n, dtype=np.uint64).astype(np.uint32)
                         for p in primes])
    b1, a1, b2, a2 = uni(q), uni(q), uni(q), uni(q)
    beta = 2
    kb = np.stack([uni(main + aux) for _ in range(beta)])
    ka = np.stack([uni(main + aux) for _ in range(beta)])
    for rs in (0, 1):
        got = chain.hmult(b1, a1, b2, a2, kb, ka, level, rs)
        want = _orc.hmult(b1, a1, b2, a2, kb, ka, L, 6, main, aux, log_n, rs)
        assert np.array_equal(got[0], want[0]) and np.array_equal(got[1],
                                                                  want[1])
    got = chain.mult_key(b1, a1, kb, ka, level)
    want = _orc.mult_key(b1, a1, kb, ka, L, 6, main, aux, log_n)
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
    got = chain.hrot(b1, a1, kb, ka, level, 3)
    want = _orc.hrot(b1, a1, kb, ka, L, 6, main, aux, log_n, 3)
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
    got = chain.rescale(b1, level)
    assert np.array_equal(got, _orc.rescale(b1, main, L, 1, log_n))


# ------------------------------------------------- terminal-prime semantics
LOG_N_SEM = 10
# main 4, terminal 3, aux 3; levels (0,2) < (2,0) < (1,3) < (4,3): going
# down drops 3 main, then 3 terminal restoring 1 main, then 2 main
# restoring 2 terminal (the pattern of parameters/bootparam_40.json)
LEVELS = [(0, 2), (2, 0), (1, 3), (4, 3)]


@pytest.fixture(scope="module")
def sem():
    chain = Chain(Q30[:4], Q25[:3], Q31[:3], LEVELS, LOG_N_SEM)
    keys = ck.Keys(LOG_N_SEM, chain.chain, chain.aux, seed=7)
    relin = keys.mult_key(chain.max_q)
    return chain, keys, relin


def _level_s(keys, chain, level):
    off = chain.offset(level)
    return keys.s_ntt[off: off + len(chain.q(level))]


def _decrypt(keys, chain, level, b, a):
    q = chain.q(level)
    v = keys._add(b, keys._mul(a, _level_s(keys, chain, level), q), q)
    return ck.from_ntt_mont(v, q, chain.log_n)


def _encrypt(keys, chain, level, m):
    q = chain.q(level)
    a = keys.uniform(q)
    e = keys.small()
    me = [int(x) + int(y) for x, y in zip(m, e)]
    b = keys._add(keys._neg(keys._mul(a, _level_s(keys, chain, level), q), q),
                  keys.ntt_of(me, q), q)
    return b, a


def _ratio(chain, level):
    """scale change of Rescale from level to level - 1 as (num, den)"""
    q_up, q_lo = chain.q(level), chain.q(level - 1)
    den = math.prod(p for p in q_up if p not in q_lo)
    num = math.prod(p for p in q_lo if p not in q_up)
    return num, den


def test_hmult_and_rescales_across_terminal_levels_decrypt(sem):
    chain, keys, (kb, ka) = sem
    n = 1 << LOG_N_SEM
    r = rng(90)
    m1, m2 = _rand_poly(r, n, 70), _rand_poly(r, n, 70)
    top = len(LEVELS) - 1
    c1, c2 = _encrypt(keys, chain, top, m1), _encrypt(keys, chain, top, m2)
    prod = ck.negacyclic_mul(m1, m2)
    b, a = chain.hmult(*c1, *c2, kb, ka, top, 1)
    want = [int(v) for v in prod]
    num, den = _ratio(chain, top)
    want = [v * num / den for v in want]
    got = _decrypt(keys, chain, top - 1, b, a)
    assert max(abs(g - w) for g, w in zip(got, want)) < 2 ** 12
    for level in (top - 1, top - 2):
        num, den = _ratio(chain, level)
        b = chain.rescale(b, level)
        a = chain.rescale(a, level)
        want = [w * num / den for w in want]
        got = _decrypt(keys, chain, level - 1, b, a)
        err = max(abs(g - w) for g, w in zip(got, want))
        assert err < 2 ** 12, (level, err)


@pytest.mark.parametrize("level", [1, 2])
def test_hrot_at_offset_levels_decrypts(sem, level):
    chain, keys, _ = sem
    n = 1 << LOG_N_SEM
    r = rng(100 + level)
    rot = 5
    g = _orc.lib.orc_galois_factor(rot, LOG_N_SEM)
    kb, ka = keys.rot_key(g, chain.max_q)
    m = _rand_poly(r, n, 40)
    b, a = _encrypt(keys, chain, level, m)
    rb, ra = chain.hrot(b, a, kb, ka, level, rot)
    want = ck.automorphism(m, g)
    got = _decrypt(keys, chain, level, rb, ra)
    assert max(abs(int(x) - int(y)) for x, y in zip(got, want)) < 2 ** 12
