"""End-to-end semantic tests on the GPU in the shape of the reference's
unittest/BasicTest.cpp (HMult merged and non-merged with a separate
Rescale, :327-374; HRot with r = 1234, :376-399; the encode / encrypt
round trips, the element-wise ciphertext ops and HConj, :10-325 and
:401-419): messages encoded by the
library, encrypted on the host under a known ternary secret (the
structure of UserInterface.cu:366-458), key-switched on the GPU at the full
N = 2^16 config-4 chain (24 main primes, 8 aux primes, dnum 3), decrypted
on the host in the NTT domain and decoded by the library, against numpy
within the reference's 1e-3 (Testbed.h:93). The residues of the same
operations are pinned bit-exactly against the oracle elsewhere
(test_gpu_parity.py); these tests check what the reference's own tests
check: that the results decrypt to the right messages."""
import os

import numpy as np
import pytest

import _orc
from gpu_util import N, config4, dev, host, zeros

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(400)]

DELTA = 2.0 ** 30
SLOTS = N // 2
L = 24


@pytest.fixture(scope="module")
def sem():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("no HIP device visible")
    import cheddar_amd
    import ckks_host as ck
    main, aux, levels = config4()
    ctx = cheddar_amd.Context(cheddar_amd.Param(main, aux, levels))
    keys = ck.Keys(16, main, aux, seed=0x5E3A)
    mk = keys.mult_key_ntt(24, rng=np.random.default_rng(0x5E3B))
    g = _orc.lib.orc_galois_factor(1234, 16)
    rk = keys.rot_key(g, 24, rng=np.random.default_rng(0x5E3C))
    ck_ = keys.rot_key(2 * N - 1, 24, rng=np.random.default_rng(0x5E3D))
    dk = lambda k: ([dev(t) for t in k[0]], [dev(t) for t in k[1]])
    return dict(ctx=ctx, keys=keys, main=main, mk=dk(mk), rk=dk(rk),
                ck=dk(ck_))


def _encrypt(s, msg, level, scale):
    """(b, a) on the device: b = -a s + Encode(msg) + e over num_q(level)"""
    ctx, keys = s["ctx"], s["keys"]
    q = s["main"][:level + 1]
    pt = zeros(level + 1, N)
    ctx.encode(level, 0, scale, msg, pt)
    a = keys.uniform(q)
    b = keys._add(keys._add(keys._neg(keys._mul(a, keys.s_ntt[:level + 1], q),
                                      q), host(pt), q),
                  keys.ntt_of(keys.small(), q), q)
    return dev(b), dev(a)


def _decrypt(s, ct, level, scale):
    """decode(b + a s) by the library"""
    keys = s["keys"]
    q = s["main"][:level + 1]
    v = keys._add(host(ct[0]), keys._mul(host(ct[1]), keys.s_ntt[:level + 1],
                                         q), q)
    return s["ctx"].decode(level, scale, SLOTS, dev(v))


def _msg(seed):
    r = np.random.default_rng(seed)
    return (r.uniform(-1, 1, SLOTS) + 1j * r.uniform(-1, 1, SLOTS))


@pytest.mark.parametrize("level", [L - 1, 12, 2])
def test_hmult_merged_rescale_decrypts(sem, level):
    """BasicTest's HMult loops over the levels; here the top one, a middle
    one and the lowest whose modulus (3 primes) holds the scale^2 product"""
    m1, m2 = _msg(1), _msg(2)
    c1 = _encrypt(sem, m1, level, DELTA)
    c2 = _encrypt(sem, m2, level, DELTA)
    res = (zeros(level, N), zeros(level, N))
    sem["ctx"].hmult(level, res, c1, c2, *sem["mk"], rescale=True)
    scale = DELTA * DELTA / sem["main"][level]
    got = _decrypt(sem, res, level - 1, scale)
    assert np.max(np.abs(got - m1 * m2)) < 1e-3


def test_hmult_then_rescale_decrypts(sem):
    m1, m2 = _msg(3), _msg(4)
    c1 = _encrypt(sem, m1, L - 1, DELTA)
    c2 = _encrypt(sem, m2, L - 1, DELTA)
    full = (zeros(L, N), zeros(L, N))
    sem["ctx"].hmult(L - 1, full, c1, c2, *sem["mk"], rescale=False)
    got = _decrypt(sem, full, L - 1, DELTA * DELTA)
    assert np.max(np.abs(got - m1 * m2)) < 1e-3
    res = (zeros(L - 1, N), zeros(L - 1, N))
    sem["ctx"].rescale(L - 1, res, full)
    got = _decrypt(sem, res, L - 2, DELTA * DELTA / sem["main"][L - 1])
    assert np.max(np.abs(got - m1 * m2)) < 1e-3


@pytest.mark.parametrize("level", [L - 1, 11])
def test_hrot_1234_decrypts(sem, level):
    m = _msg(5)
    c = _encrypt(sem, m, level, DELTA)
    res = (zeros(level + 1, N), zeros(level + 1, N))
    sem["ctx"].hrot(level, res, c, *sem["rk"], 1234)
    got = _decrypt(sem, res, level, DELTA)
    assert np.max(np.abs(got - np.roll(m, -1234))) < 1e-3


# --------------------------------------------------------------------------
# the rest of BasicTest at config 4 (BasicTest.cpp:10-325, 401-419): encode /
# encrypt round trips, the ciphertext-ciphertext, -plaintext and -constant
# ops through chd_elementwise composed as Context::Add / Sub / Neg / Mult /
# MultImaginaryUnit compose them (Context.cpp; b op operand, a copied for a
# plaintext or constant operand), and HConj = MultKey with the conjugation
# key, then PermuteConjugate (Context.cpp:794-798). Two levels: the top one
# and one whose modulus (4 primes) still holds a product at scale 2^60.
# --------------------------------------------------------------------------
BASIC_LEVELS = [L - 1, 3]


def _ct(level):
    return (zeros(level + 1, N), zeros(level + 1, N))


def _pt(s, msg, level, scale=DELTA):
    pt = zeros(level + 1, N)
    s["ctx"].encode(level, 0, scale, msg, pt)
    return pt


def _const(s, value, level, scale=DELTA):
    cx = zeros(level + 1)
    s["ctx"].encode_constant(level, 0, scale, value, cx)
    return cx


@pytest.mark.parametrize("level", BASIC_LEVELS)
def test_encode_decode_and_encrypt_decrypt(sem, level):
    m = _msg(20)
    got = sem["ctx"].decode(level, DELTA, SLOTS, _pt(sem, m, level))
    assert np.max(np.abs(got - m)) < 1e-3
    got = _decrypt(sem, _encrypt(sem, m, level, DELTA), level, DELTA)
    assert np.max(np.abs(got - m)) < 1e-3


@pytest.mark.parametrize("level", BASIC_LEVELS)
@pytest.mark.parametrize("op", ["add", "sub"])
def test_ct_ct_add_sub_decrypts(sem, level, op):
    m1, m2 = _msg(21), _msg(22)
    c1, c2 = _encrypt(sem, m1, level, DELTA), _encrypt(sem, m2, level, DELTA)
    res = _ct(level)
    sem["ctx"].elementwise(level, 0, op, list(res), list(c1), list(c2))
    want = m1 + m2 if op == "add" else m1 - m2
    assert np.max(np.abs(_decrypt(sem, res, level, DELTA) - want)) < 1e-3


@pytest.mark.parametrize("level", BASIC_LEVELS)
@pytest.mark.parametrize("op", ["add", "sub"])
def test_ct_pt_add_sub_decrypts(sem, level, op):
    m1, m2 = _msg(23), _msg(24)
    c1 = _encrypt(sem, m1, level, DELTA)
    res = _ct(level)
    sem["ctx"].elementwise(level, 0, op, [res[0]], [c1[0]],
                           [_pt(sem, m2, level)])
    sem["ctx"].elementwise(level, 0, "copy", [res[1]], [c1[1]])
    want = m1 + m2 if op == "add" else m1 - m2
    assert np.max(np.abs(_decrypt(sem, res, level, DELTA) - want)) < 1e-3


@pytest.mark.parametrize("level", BASIC_LEVELS)
@pytest.mark.parametrize("op", ["add_const", "sub_const"])
def test_ct_const_add_sub_decrypts(sem, level, op):
    m1 = _msg(25)
    value = _msg(26)[0].real
    c1 = _encrypt(sem, m1, level, DELTA)
    res = _ct(level)
    sem["ctx"].elementwise(level, 0, op, [res[0]], [c1[0]],
                           cst=_const(sem, value, level))
    sem["ctx"].elementwise(level, 0, "copy", [res[1]], [c1[1]])
    want = m1 + value if op == "add_const" else m1 - value
    assert np.max(np.abs(_decrypt(sem, res, level, DELTA) - want)) < 1e-3


@pytest.mark.parametrize("level", BASIC_LEVELS)
def test_neg_ct_decrypts(sem, level):
    m1 = _msg(27)
    c1 = _encrypt(sem, m1, level, DELTA)
    res = _ct(level)
    sem["ctx"].elementwise(level, 0, "neg", list(res), list(c1))
    assert np.max(np.abs(_decrypt(sem, res, level, DELTA) + m1)) < 1e-3


@pytest.mark.parametrize("level", BASIC_LEVELS)
def test_ct_mult_pt_and_const_decrypt(sem, level):
    """without rescaling: the products decrypt at scale^2"""
    m1, m2 = _msg(28), _msg(29)
    value = _msg(30)[0].real
    c1 = _encrypt(sem, m1, level, DELTA)
    res = _ct(level)
    sem["ctx"].elementwise(level, 0, "pmult", list(res), list(c1),
                           [_pt(sem, m2, level)])
    got = _decrypt(sem, res, level, DELTA * DELTA)
    assert np.max(np.abs(got - m1 * m2)) < 1e-3
    sem["ctx"].elementwise(level, 0, "mult_const", list(res), list(c1),
                           cst=_const(sem, value, level))
    got = _decrypt(sem, res, level, DELTA * DELTA)
    assert np.max(np.abs(got - m1 * value)) < 1e-3


@pytest.mark.parametrize("level", BASIC_LEVELS)
def test_ct_mult_imaginary_unit_decrypts(sem, level):
    m1 = _msg(31)
    c1 = _encrypt(sem, m1, level, DELTA)
    res = _ct(level)
    sem["ctx"].elementwise(level, 0, "mult_i", list(res), list(c1))
    assert np.max(np.abs(_decrypt(sem, res, level, DELTA) - 1j * m1)) < 1e-3


@pytest.mark.parametrize("level", BASIC_LEVELS)
def test_hconj_decrypts(sem, level):
    m1 = _msg(32)
    c1 = _encrypt(sem, m1, level, DELTA)
    tmp, res = _ct(level), _ct(level)
    sem["ctx"].mult_key(level, tmp, c1, *sem["ck"])
    sem["ctx"].permute(level, res, tmp, -1)
    got = _decrypt(sem, res, level, DELTA)
    assert np.max(np.abs(got - np.conj(m1))) < 1e-3


# --------------------------------------------------------------------------
# the reference's parameter files, as BasicTest is instantiated
# (BasicTest.cpp:421-429): terminal primes, 20-bit primes, two-prime rescales
# --------------------------------------------------------------------------
PARAMS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "params")


@pytest.fixture(scope="module", params=["bootparam_30.json",
                                        "bootparam_35.json",
                                        "bootparam_40.json"])
def tsem(request):
    import json
    import torch
    if not torch.cuda.is_available():
        pytest.fail("no HIP device visible")
    import cheddar_amd
    import ckks_host as ck
    from ks_ref import Chain
    _orc.lib.orc_set_threads(16)
    text = open(os.path.join(PARAMS, request.param)).read()
    d = json.loads(text)
    ctx = cheddar_amd.Context(cheddar_amd.Param.from_json(text))
    chain = Chain(d["main_primes"], d["terminal_primes"],
                  d["auxiliary_primes"], d["level_config"], 16)
    keys = ck.Keys(16, chain.chain, chain.aux, seed=0x7E5)
    dk = lambda k: ([dev(t) for t in k[0]], [dev(t) for t in k[1]])
    mk = dk(keys.mult_key_ntt(chain.max_q, rng=np.random.default_rng(1)))
    g = _orc.lib.orc_galois_factor(1234, 16)
    rk = dk(keys.rot_key(g, chain.max_q, rng=np.random.default_rng(2)))
    print("parameter set", request.param, flush=True)
    return dict(ctx=ctx, chain=chain, keys=keys, mk=mk, rk=rk,
                level=d["default_encryption_level"],
                scale=2.0 ** d["log_default_scale"])


def _t_s(t, level):
    off = t["chain"].offset(level)
    return t["keys"].s_ntt[off: off + len(t["chain"].q(level))]


def _t_encrypt(t, msg, level):
    keys, q = t["keys"], t["chain"].q(level)
    pt = zeros(len(q), N)
    t["ctx"].encode(level, 0, t["scale"], msg, pt)
    a = keys.uniform(q)
    b = keys._add(keys._add(keys._neg(keys._mul(a, _t_s(t, level), q), q),
                            host(pt), q), keys.ntt_of(keys.small(), q), q)
    return dev(b), dev(a)


def _t_decrypt(t, ct, level, scale):
    keys, q = t["keys"], t["chain"].q(level)
    v = keys._add(host(ct[0]), keys._mul(host(ct[1]), _t_s(t, level), q), q)
    return t["ctx"].decode(level, scale, SLOTS, dev(v))


def test_param_files_hmult_decrypts(tsem):
    """HMult with the merged rescale at the default encryption level: the
    result's scale is scale^2 times the primes the rescale restores over
    the ones it drops"""
    import math
    chain, lv = tsem["chain"], tsem["level"]
    m1, m2 = _msg(11), _msg(12)
    c1, c2 = _t_encrypt(tsem, m1, lv), _t_encrypt(tsem, m2, lv)
    nq = len(chain.q(lv - 1))
    res = (zeros(nq, N), zeros(nq, N))
    tsem["ctx"].hmult(lv, res, c1, c2, *tsem["mk"], rescale=True)
    up, lo = chain.q(lv), chain.q(lv - 1)
    num = math.prod(p for p in lo if p not in up)
    den = math.prod(p for p in up if p not in lo)
    got = _t_decrypt(tsem, res, lv - 1, tsem["scale"] ** 2 * num / den)
    assert np.max(np.abs(got - m1 * m2)) < 1e-3


def test_param_files_hrot_1234_decrypts(tsem):
    lv = tsem["level"]
    m = _msg(13)
    c = _t_encrypt(tsem, m, lv)
    nq = len(tsem["chain"].q(lv))
    res = (zeros(nq, N), zeros(nq, N))
    tsem["ctx"].hrot(lv, res, c, *tsem["rk"], 1234)
    got = _t_decrypt(tsem, res, lv, tsem["scale"])
    assert np.max(np.abs(got - np.roll(m, -1234))) < 1e-3
