"""CPU tests that pin the oracle before it is trusted as the parity checker.

Pins, in order: the reference's own constant recipe (fixture from the
reference headers, and live when /root/reference is present), closed-form
DFT, independent exact-vs-faithful NTT paths, convolution theorem, exact CRT
for BConv, fast-base-conversion invariants for ModUp, known answers for
ModDown/Rescale, algebraic identities for Tensor/PAccum/Permute, and finally
semantic decryption of HMult/HRot outputs under a known secret.
"""
import json
import os
import random
import shutil
import subprocess

import numpy as np
import pytest

import _orc
import ckks_host as ck
from chd_primes import ntt_primes

HERE = os.path.dirname(os.path.abspath(__file__))
R = 1 << 32
Q30 = ntt_primes(30, 32)
Q31 = ntt_primes(31, 16)
CFG1_Q = 2147352577


def brev(i, bits):
    return int(format(i, "0%db" % bits)[::-1], 2)


def rng(seed):
    return np.random.default_rng(seed)


def uniform(r, q, n):
    return r.integers(0, q, n, dtype=np.uint64).astype(np.uint32)


# --------------------------------------------------------------------------
# constants
# --------------------------------------------------------------------------
def _check_case(case):
    log_n = case["log_n"]
    n = 1 << log_n
    idx = [0, 1, 2, 3, 5, 255, 256, 4097, n // 2 + 7, n - 1]
    for row, tw in zip(case["primes"], case["tw"]):
        q, g, psi, qinv, ninv, ninv_m, r2 = row
        pr, pir, c = _orc.twiddles(q, log_n)
        assert int(c[4]) == g and int(c[3]) == psi
        assert _orc.lib.orc_inv_mod_base(q) == qinv
        assert [int(c[0]), int(c[1]), int(c[2])] == [ninv, ninv_m, r2]
        for k, j in enumerate(idx):
            if j < n:
                assert int(pr[j]) == tw[2 * k] and int(pir[j]) == tw[2 * k + 1]
    c1, c2 = _orc.modswitch_consts(case["src"], case["dst"], log_n)
    assert c1.tolist() == case["const1"]
    assert c2.reshape(-1).tolist() == case["const2"]
    inv, _ = _orc.moddown_consts(case["src"], case["dst"])
    assert inv.tolist() == case["invpp"]


def test_constants_match_reference_fixture():
    with open(os.path.join(HERE, "golden", "ref_constants.json")) as f:
        fx = json.load(f)
    for case in fx["cases"]:
        _check_case(case)


def test_constants_match_live_reference():
    """Rebuilds refcheck from /root/reference (this container only)."""
    if not os.path.isdir("/root/reference/include") or not shutil.which("g++"):
        pytest.skip("reference tree not present")
    root = os.path.dirname(HERE)
    subprocess.check_call(["make", "-s", "-C", os.path.join(root, "oracle"),
                           "ref"])
    src = ntt_primes(31, 3, skip=9)
    dst = ntt_primes(30, 5, skip=20)
    out = subprocess.check_output(
        [os.path.join(root, "oracle", "_ref", "refcheck"), "13",
         str(len(src)), str(len(dst))] + [str(p) for p in src + dst],
        text=True)
    import golden.make_golden as mg  # noqa: E402
    case = mg.parse(out)
    case.update(log_n=13, src=src, dst=dst)
    _check_case(case)


def test_config1_prime_constants():
    _, _, c = _orc.twiddles(CFG1_Q, 16)
    assert int(c[4]) == 5 and int(c[3]) == 1615402923
    psi = int(c[3])
    assert pow(psi, 1 << 16, CFG1_Q) == CFG1_Q - 1   # psi^N = -1
    assert pow(psi, 1 << 17, CFG1_Q) == 1


@pytest.mark.parametrize("q", [7681, 12289, 40961, 65537, 786433])
def test_generator_is_smallest(q):
    def order_is_full(r):
        x, k = r, 1
        while x != 1:
            x = x * r % q
            k += 1
        return k == q - 1
    g = next(r for r in range(2, q) if order_is_full(r))
    assert _orc.lib.orc_find_generator(q) == g


def test_inv_mod_base_and_mont_mul():
    r = random.Random(5)
    for q in Q30[:4] + Q31[:4]:
        qi = _orc.lib.orc_inv_mod_base(q)
        assert (q * qi) % R == 1 and -(1 << 31) <= qi < (1 << 31)
        for _ in range(50):
            a, b = r.randrange(q), r.randrange(q)
            m = _orc.lib.orc_mont_mul(a, b, q)
            assert 0 <= m < q and (m * R - a * b) % q == 0


# --------------------------------------------------------------------------
# NTT
# --------------------------------------------------------------------------
def dft(x, q, log_n, rows):
    n = 1 << log_n
    psi = _orc.lib.orc_primitive_root(2 * n, q)
    pw = [1] * (2 * n)
    for k in range(1, 2 * n):
        pw[k] = pw[k - 1] * psi % q
    xs = [int(v) for v in x]
    out = []
    for i in rows:
        e = 2 * brev(i, log_n) + 1
        out.append(sum(xs[j] * pw[(e * j) % (2 * n)] for j in range(n)) % q)
    return out


@pytest.mark.parametrize("log_n", [3, 5, 8])
@pytest.mark.parametrize("mont", [0, 1])
def test_ntt_closed_form_small(log_n, mont):
    q = Q31[1]
    x = uniform(rng(log_n), q, 1 << log_n)
    want = dft([int(v) * (R if mont else 1) % q for v in x], q, log_n,
               range(1 << log_n))
    assert _orc.ntt(x, log_n, q, mont, exact=True).tolist() == want
    assert _orc.ntt(x, log_n, q, mont).tolist() == want


def test_ntt_closed_form_sampled_2_16():
    for q in (CFG1_Q, Q30[0]):
        x = uniform(rng(q), q, 1 << 16)
        rows = [0, 1, 2, 12345, 32768, 65535]
        y = _orc.ntt(x, 16, q, 0)
        # vectorised closed form for the sampled rows
        n = 1 << 16
        psi = _orc.lib.orc_primitive_root(2 * n, q)
        pw = np.ones(2 * n, np.uint64)
        for k in range(1, 2 * n):
            pw[k] = pw[k - 1] * np.uint64(psi) % np.uint64(q)
        j = np.arange(n, dtype=np.uint64)
        for i in rows:
            e = np.uint64(2 * brev(i, 16) + 1)
            terms = x.astype(np.uint64) * pw[(e * j) % np.uint64(2 * n)] % \
                np.uint64(q)
            assert int(terms.sum() % np.uint64(q)) == int(y[i])


@pytest.mark.parametrize("q", [CFG1_Q, Q31[7], Q30[0], Q30[31]])
def test_faithful_equals_exact_and_roundtrip(q):
    x = uniform(rng(q % 1000), q, 1 << 16)
    for mont in (0, 1):
        a = _orc.ntt(x, 16, q, mont)
        assert np.array_equal(a, _orc.ntt(x, 16, q, mont, exact=True))
        assert a.max() < q
        b = _orc.intt(a, 16, q, mont)
        assert np.array_equal(b, _orc.intt(a, 16, q, mont, exact=True))
        assert np.array_equal(b, x)      # mc pairing returns the input
    # intt(mc=1) of a plain NTT is x * R^-1
    y = _orc.intt(_orc.ntt(x, 16, q, 0), 16, q, 1)
    assert np.array_equal(y.astype(np.uint64) * (R % q) % q, x)


def test_negacyclic_convolution_theorem():
    log_n, q = 8, Q30[3]
    r = rng(9)
    a = uniform(r, q, 256)
    b = uniform(r, q, 256)
    fa = _orc.ntt(a, log_n, q, 0).astype(np.uint64)
    fb = _orc.ntt(b, log_n, q, 0).astype(np.uint64)
    c = _orc.intt((fa * fb % q).astype(np.uint32), log_n, q, 0)
    want = ck.negacyclic_mul([int(v) for v in a], [int(v) for v in b])
    assert c.tolist() == [int(v) % q for v in want]


def test_intt_mult_const_centred():
    log_n, q = 10, Q31[2]
    x = uniform(rng(3), q, 1 << log_n)
    cst = 123456789 % q
    out = _orc.intt_mult_const(x, log_n, q, cst, 1)
    plain = _orc.intt(x, log_n, q, 0, exact=True).astype(object)
    n = 1 << log_n
    want = [(int(v) * n * cst * pow(R, -1, q)) % q for v in plain]
    half = (q - 1) // 2
    assert all(-half <= int(v) <= half for v in out)
    assert [int(v) % q for v in out] == want


# --------------------------------------------------------------------------
# BConv / ModUp / ModDown
# --------------------------------------------------------------------------
def test_bconv_exact_crt():
    log_n = 10
    src = Q30[:8]
    dst = Q31[:12]
    c1, table = _orc.modswitch_consts(src, dst, log_n)
    r = rng(11)
    cent = np.stack([r.integers(-(q - 1) // 2, (q - 1) // 2 + 1, 1 << log_n)
                     for q in src]).astype(np.int32)
    out = _orc.bconv(cent, table, dst, log_n)
    Q = 1
    for q in src:
        Q *= q
    qhat = [Q // q for q in src]
    for n_ in (0, 1, 777, 1023):
        X = sum(int(cent[i, n_]) * qhat[i] for i in range(len(src)))
        for k, p in enumerate(dst):
            assert int(out[k, n_]) == X * R % p


def test_mod_up_invariants():
    log_n, alpha = 10, 2
    qp, pp = Q30[:5], Q31[:alpha]
    L = len(qp)
    primes = qp + pp
    x = np.stack([uniform(rng(20 + i), q, 1 << log_n)
                  for i, q in enumerate(qp)])
    out = _orc.mod_up(x, qp, pp, log_n)
    assert out.shape[0] == 3
    coef = _orc.intt_batch(x.reshape(-1), log_n, qp, 1).reshape(L, -1)
    for g in range(3):
        s, e = g * alpha, min((g + 1) * alpha, L)
        grp = qp[s:e]
        Qg = 1
        for q in grp:
            Qg *= q
        assert np.array_equal(out[g, s:e], x[s:e])     # own limbs copied
        oc = _orc.intt_batch(out[g].reshape(-1), log_n, primes, 1).reshape(
            L + alpha, -1)
        for n_ in (0, 5, 1023):
            X = 0
            for i, q in enumerate(grp):
                qh = Qg // q
                v = int(coef[s + i, n_]) * pow(qh % q, -1, q) % q
                if v > q // 2:
                    v -= q
                X += v * qh
            assert abs(X) <= len(grp) * Qg // 2
            for j, p in enumerate(primes):
                assert int(oc[j, n_]) == X % p


def _kat_input(log_n, q_primes, divisor, r):
    n = 1 << log_n
    Y = [int(v) for v in r.integers(-(1 << 40), 1 << 40, n)]
    Z = [v * divisor for v in Y]
    return Y, Z


@pytest.mark.parametrize("kind", ["moddown", "rescale", "merged"])
def test_mod_down_known_answer(kind):
    log_n, alpha = 10, 2
    qp, pp = Q30[:4], Q31[:alpha]
    L = len(qp)
    P = pp[0] * pp[1]
    r = rng(31)
    if kind == "moddown":
        primes, keep, div = qp + pp, L, P
    elif kind == "rescale":
        primes, keep, div = qp, L - 1, qp[-1]
    else:
        primes, keep, div = qp + pp, L - 1, qp[-1] * P
    Y, Z = _kat_input(log_n, qp, div, r)
    src = ck.to_ntt_mont(Z, primes, log_n)
    out = _orc.mod_down(src, primes, keep, log_n)
    want = ck.to_ntt_mont(Y, qp[:keep], log_n)
    assert np.array_equal(out, want)


@pytest.mark.parametrize("kind", ["moddown", "rescale", "merged"])
def test_mod_down_rounding_bound(kind):
    """Random input: out * D = Z - X (mod Q_out) with |X| <= s D / 2, D the
    product of the s primes divided out (P, q_top, or q_top P): each dropped
    prime contributes its centred residue times D / d_i."""
    log_n, alpha = 8, 3
    qp, pp = Q30[:8], Q31[:alpha]
    if kind == "moddown":
        primes, keep, dropped = qp + pp, len(qp), pp
    elif kind == "rescale":
        primes, keep, dropped = qp, len(qp) - 1, qp[-1:]
    else:
        primes, keep, dropped = qp + pp, len(qp) - 1, qp[-1:] + pp
    D = 1
    for d in dropped:
        D *= d
    Q = 1
    for q in qp[:keep]:
        Q *= q
    assert len(dropped) * D < Q >> 60  # the bound says something mod Q
    src = np.stack([uniform(rng(40 + i), p, 1 << log_n)
                    for i, p in enumerate(primes)])
    out = _orc.mod_down(src, primes, keep, log_n)
    Zc = ck.from_ntt_mont(src[:keep], qp[:keep], log_n)
    Yc = ck.from_ntt_mont(out, qp[:keep], log_n)
    worst = 0
    for z, y in zip(Zc, Yc):
        d = (z - y * D) % Q
        if d > Q // 2:
            d -= Q
        assert abs(d) <= len(dropped) * D // 2
        worst = max(worst, abs(d))
    # the bound is not slack by orders of magnitude: X really is of size D
    assert worst > D // 16


# --------------------------------------------------------------------------
# element-wise
# --------------------------------------------------------------------------
def test_tensor_identity():
    log_n = 8
    qs = Q30[:3]
    r = rng(50)
    b1, a1, b2, a2 = (np.stack([uniform(r, q, 256) for q in qs])
                      for _ in range(4))
    bx, ax, rx = _orc.tensor(b1, a1, b2, a2, qs, log_n)
    for i, q in enumerate(qs):
        s = uniform(r, q, 256).astype(object)
        lhs = ((b1[i].astype(object) + a1[i].astype(object) * s) *
               (b2[i].astype(object) + a2[i].astype(object) * s))
        rhs = (bx[i].astype(object) + ax[i].astype(object) * s +
               rx[i].astype(object) * s * s) * R
        assert all(int(v) % q == 0 for v in (lhs - rhs))


def test_paccum_caccum_direct_sum():
    log_n, alpha, L, max_q = 6, 2, 3, 5
    qs, ps = Q30[:max_q], Q31[:alpha]
    beta = 2
    primes = qs[:L] + ps
    r = rng(60)
    n = 1 << log_n
    modup = np.stack([np.stack([uniform(r, p, n) for p in primes])
                      for _ in range(beta)])
    kp = qs + ps
    kb = np.stack([np.stack([uniform(r, p, n) for p in kp])
                   for _ in range(beta)])
    ka = np.stack([np.stack([uniform(r, p, n) for p in kp])
                   for _ in range(beta)])
    acc_b = np.zeros((L + alpha, n), np.uint32)
    acc_a = np.zeros_like(acc_b)
    _orc.lib.orc_paccum(acc_b, acc_a, modup, beta, kb, ka, L, alpha, max_q,
                        _orc.u32(primes), log_n)
    for l, p in enumerate(primes):
        kl = l if l < L else max_q + l - L
        want = sum(modup[g, l].astype(object) * kb[g, kl].astype(object)
                   for g in range(beta))
        want = [int(v) * pow(R, -1, p) % p for v in want]
        assert acc_b[l].tolist() == want
    # order independence over the dnum groups
    acc2 = np.zeros_like(acc_b)
    acc2a = np.zeros_like(acc_b)
    _orc.lib.orc_paccum(acc2, acc2a, np.ascontiguousarray(modup[::-1]), beta,
                        np.ascontiguousarray(kb[::-1]),
                        np.ascontiguousarray(ka[::-1]), L, alpha, max_q,
                        _orc.u32(primes), log_n)
    assert np.array_equal(acc2, acc_b) and np.array_equal(acc2a, acc_a)
    pprod = _orc.p_prod(qs[:L], ps)
    ct = np.stack([uniform(r, p, n) for p in qs[:L]])
    before = acc_b.copy()
    _orc.lib.orc_caccum(acc_b, ct, pprod, L, _orc.u32(primes), log_n)
    P = ps[0] * ps[1]
    for l in range(L):
        q = qs[l]
        want = (before[l].astype(object) + ct[l].astype(object) * P) % q
        assert acc_b[l].tolist() == [int(v) for v in want]
    assert np.array_equal(acc_b[L:], before[L:])


def test_pmult_accum_direct_sum():
    """the giant-step plaintext accumulation: acc = sum_b pt_b x_b R^-1 mod p
    with Python integers, including the residues 0 and p - 1, and the same
    result with threads"""
    log_n = 7
    primes = Q30[:3] + Q31[:2]
    n = 1 << log_n
    r = rng(65)
    terms = [(np.stack([uniform(r, p, n) for p in primes]),
              np.stack([uniform(r, p, n) for p in primes])) for _ in range(5)]
    for l, p in enumerate(primes):  # extreme residues in the first columns
        terms[0][0][l, :2] = (0, p - 1)
        terms[0][1][l, :2] = (p - 1, p - 1)
    outs = []
    for threads in (1, 4):
        _orc.lib.orc_set_threads(threads)
        acc = np.zeros((len(primes), n), np.uint32)
        for pt, x in terms:
            _orc.pmult_accum(acc, pt, x, primes, log_n)
        outs.append(acc)
    _orc.lib.orc_set_threads(1)
    for l, p in enumerate(primes):
        want = sum(pt[l].astype(object) * x[l].astype(object)
                   for pt, x in terms)
        assert outs[0][l].tolist() == [int(v) * pow(R, -1, p) % p
                                       for v in want]
    assert np.array_equal(outs[0], outs[1])


def test_permute_composition_and_coefficient_map():
    log_n = 8
    q = Q30[5]
    n = 1 << log_n
    x = uniform(rng(70), q, n)
    y = _orc.ntt(x, log_n, q, 0)
    g1 = _orc.lib.orc_galois_factor(3, log_n)
    g2 = _orc.lib.orc_galois_factor(5, log_n)
    assert g1 == pow(5, 3, 2 * n)
    both = _orc.permute(_orc.permute(y, log_n, g2), log_n, g1)
    assert np.array_equal(both, _orc.permute(y, log_n, g1 * g2 % (2 * n)))
    for g in (g1, 2 * n - 1):
        want = ck.automorphism([int(v) for v in x], g)
        want = np.array([int(v) % q for v in want], np.uint32)
        assert np.array_equal(_orc.permute(y, log_n, g),
                              _orc.ntt(want, log_n, q, 0))


# --------------------------------------------------------------------------
# key switching: semantic decryption under a known secret
# --------------------------------------------------------------------------
LOG_N_SEM = 10
DELTA = 1 << 20


@pytest.fixture(scope="module")
def sem():
    qp, pp = Q30[:6], Q31[:2]
    keys = ck.Keys(LOG_N_SEM, qp, pp, seed=3)
    max_q = 6
    kb, ka = keys.mult_key(max_q)
    return keys, kb, ka, max_q


def _message(r, n, scale):
    return [int(v) for v in r.integers(-4, 5, n) * scale]


@pytest.mark.parametrize("L", [6, 5])
def test_hmult_decrypts(sem, L):
    keys, kb, ka, max_q = sem
    r = rng(80 + L)
    n = keys.n
    m1, m2 = _message(r, n, DELTA), _message(r, n, DELTA)
    b1, a1 = keys.encrypt(m1, L)
    b2, a2 = keys.encrypt(m2, L)
    prod = ck.negacyclic_mul(m1, m2)
    # merged ModDown+Rescale
    rb, ra = _orc.hmult(b1, a1, b2, a2, kb, ka, L, max_q, keys.q, keys.p,
                        LOG_N_SEM, 1)
    dec = keys.decrypt(rb, ra, L - 1)
    qt = keys.q[L - 1]
    err = max(abs(d - int(p) / qt) for d, p in zip(dec, prod))
    assert err < 64
    # relinearize only, then a separate Rescale: same message, different bits
    sb, sa = _orc.hmult(b1, a1, b2, a2, kb, ka, L, max_q, keys.q, keys.p,
                        LOG_N_SEM, 0)
    dec0 = keys.decrypt(sb, sa, L)
    # before rescale the encryption noise times m (|e m| N ~ 2^30) dominates;
    # the product itself is ~2^50
    assert max(abs(d - int(p)) for d, p in zip(dec0, prod)) < qt * 8
    xb = _orc.rescale(sb, keys.q, L, 1, LOG_N_SEM)
    xa = _orc.rescale(sa, keys.q, L, 1, LOG_N_SEM)
    dec1 = keys.decrypt(xb, xa, L - 1)
    assert max(abs(d - int(p) / qt) for d, p in zip(dec1, prod)) < 64
    # one rounding (by q_top P) against two (by P, then by q_top): the
    # merged form is a different function, not a refactoring of the other
    assert not (np.array_equal(rb, xb) and np.array_equal(ra, xa))


def test_hrot_decrypts(sem):
    keys, _, _, max_q = sem
    L = 5
    rot = 3
    g = _orc.lib.orc_galois_factor(rot, LOG_N_SEM)
    kb, ka = keys.rot_key(g, max_q)
    r = rng(90)
    m = _message(r, keys.n, DELTA)
    b, a = keys.encrypt(m, L)
    rb, ra = _orc.hrot(b, a, kb, ka, L, max_q, keys.q, keys.p, LOG_N_SEM, rot)
    dec = keys.decrypt(rb, ra, L)
    want = ck.automorphism(m, g)
    assert max(abs(d - int(w)) for d, w in zip(dec, want)) < 1 << 12


# --------------------------------------------------------------------------
# hoisted rotations (src/extension/Hoist.cu), restated in tests/hoist_ref.py
# --------------------------------------------------------------------------
def test_hoisted_baby_step_moddown_is_hrot(sem):
    """ModDown of an extended-basis baby step is exactly HRot: the key
    switch is the same, PseudoModUp(b) = P b contributes b after the
    division by P, and the automorphism commutes with ModDown."""
    import hoist_ref
    keys, _, _, max_q = sem
    L = 5
    r = rng(95)
    b, a = keys.uniform(keys.q[:L]), keys.uniform(keys.q[:L])
    primes = keys.q[:L] + keys.p
    for rot in (1, 7):
        g = _orc.lib.orc_galois_factor(rot, LOG_N_SEM)
        kb, ka = keys.rot_key(g, max_q)
        sb, sa = hoist_ref.baby_step(b, a, (kb, ka), rot, L, max_q, keys.q,
                                     keys.p, LOG_N_SEM)
        hb, ha = _orc.hrot(b, a, kb, ka, L, max_q, keys.q, keys.p, LOG_N_SEM,
                           rot)
        assert np.array_equal(_orc.mod_down(sb, primes, L, LOG_N_SEM), hb)
        assert np.array_equal(_orc.mod_down(sa, primes, L, LOG_N_SEM), ha)
    # rotation 0: PseudoModUp of both parts, divided by P gives the input
    sb, sa = hoist_ref.baby_step(b, a, None, 0, L, max_q, keys.q, keys.p,
                                 LOG_N_SEM)
    assert np.array_equal(_orc.mod_down(sb, primes, L, LOG_N_SEM), b)
    assert np.array_equal(_orc.mod_down(sa, primes, L, LOG_N_SEM), a)
    assert not sb[L:].any() and not sa[L:].any()


def test_hoisted_bsgs_decrypts(sem):
    """sum_g Rot_g(sum_b pt[g,b] * Rot_b(m)), rescaled, decrypts to the
    plaintext-domain result under the known secret."""
    import hoist_ref
    keys, _, _, max_q = sem
    L = 6
    n = keys.n
    r = rng(96)
    m = [int(v) for v in r.integers(-4, 5, n) * (1 << 30)]
    b, a = keys.encrypt(m, L)
    primes = keys.q[:L] + keys.p
    bsi, gsi = (0, 1, 2), (0, 3)
    pts, pt_coef = {}, {}
    for g in gsi:
        for s in bsi:
            c = [int(v) for v in r.integers(-2, 3, n)]
            pt_coef[(g, s)] = c
            pts[(g, s)] = keys.ntt_of(c, primes)
    rot_keys = {}
    for rot in (1, 2, 3):
        rot_keys[rot] = keys.rot_key(_orc.lib.orc_galois_factor(rot, LOG_N_SEM),
                                     max_q)
    rb, ra = hoist_ref.evaluate(b, a, pts, rot_keys, L, max_q, keys.q, keys.p,
                                LOG_N_SEM)
    dec = keys.decrypt(rb, ra, L - 1)
    want = np.zeros(n, dtype=object)
    for g in gsi:
        inner = np.zeros(n, dtype=object)
        for s in bsi:
            gs_ = _orc.lib.orc_galois_factor(s, LOG_N_SEM)
            inner = inner + ck.negacyclic_mul(pt_coef[(g, s)],
                                              ck.automorphism(m, gs_))
        want = want + ck.automorphism(list(inner),
                                      _orc.lib.orc_galois_factor(g, LOG_N_SEM))
    qt = keys.q[L - 1]
    err = max(abs(d - int(w) / qt) for d, w in zip(dec, want))
    assert max(abs(int(w)) for w in want) / qt > 1 << 6  # the check is not vacuous
    assert err < 64
