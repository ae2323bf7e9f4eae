"""GPU parity of the element-wise ops (ElementWise.cu:687-920, 1673-1706:
Add, Sub, Neg, Mult, PMult, AddConst, SubConst, SubOppositeConst,
MultConst, MultImaginaryUnit, Copy) through chd_elementwise, bit-exact
against numpy modular arithmetic on canonical residues, with aux limbs, the
edge residues 0 and q - 1, one to three polynomials and dst aliasing a.

MultImaginaryUnit is pinned by what fixes it: applied twice it is Neg
exactly, and on an encoding it decodes to i * m (the sign and the slot
halves); the Context-level ops on Ciphertext objects are covered by the C++
API test (tests/cpp/test_api.cpp).
"""
import numpy as np
import pytest

from ckks_host import mont_mul_vec
from gpu_util import N, config4, dev, host, zeros

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("no HIP device visible")
    import cheddar_amd
    main, aux, levels = config4()
    return cheddar_amd.Context(cheddar_amd.Param(main, aux, levels)), main, aux


def _operand(r, primes, edge=False):
    x = np.stack([r.integers(0, p, N, dtype=np.uint64).astype(np.uint32)
                  for p in primes])
    if edge:
        for i, p in enumerate(primes):
            x[i, :64] = 0
            x[i, 64:128] = p - 1
    return x


def _const(cx, n=N):
    return np.repeat(cx[:, None], n, axis=1)


def _want(op, x, y, c, primes):
    q = np.array(primes, np.uint64)[:, None]
    x64 = x.astype(np.uint64)
    if op == "add":
        return ((x64 + y) % q).astype(np.uint32)
    if op == "sub":
        return ((x64 + q - y) % q).astype(np.uint32)
    if op == "neg":
        return ((q - x64) % q).astype(np.uint32)
    if op in ("mult", "pmult"):
        return np.stack([mont_mul_vec(x[i], y[i], p)
                         for i, p in enumerate(primes)])
    cb = _const(c).astype(np.uint64)
    if op == "add_const":
        return ((x64 + cb) % q).astype(np.uint32)
    if op == "sub_const":
        return ((x64 + q - cb) % q).astype(np.uint32)
    if op == "sub_opp_const":
        return ((cb + q - x64) % q).astype(np.uint32)
    if op == "mult_const":
        return np.stack([mont_mul_vec(x[i], _const(c[i:i + 1])[0], p)
                         for i, p in enumerate(primes)])
    assert op == "copy"
    return x


OPS = ["add", "sub", "neg", "mult", "pmult", "add_const", "sub_const",
       "sub_opp_const", "mult_const", "copy"]


@pytest.mark.parametrize("op", OPS)
@pytest.mark.parametrize("level,num_aux,num_poly", [(23, 0, 2), (7, 8, 3),
                                                    (0, 3, 1)])
def test_elementwise_op(ctx, op, level, num_aux, num_poly):
    c, main, aux = ctx
    primes = main[:level + 1] + aux[:num_aux]
    r = np.random.default_rng(hash((op, level)) % 10000)
    xs = [_operand(r, primes, edge=True) for _ in range(num_poly)]
    ys = [_operand(r, primes, edge=True) for _ in range(num_poly)]
    cx = np.array([r.integers(0, p) for p in primes], np.uint32)
    cx[0] = primes[0] - 1
    dst = [zeros(len(primes), N) for _ in range(num_poly)]
    b = [dev(y) for y in ys]
    c.elementwise(level, num_aux, op, dst, [dev(x) for x in xs],
                  b if op != "pmult" else b[:1], dev(cx))
    for p in range(num_poly):
        y = ys[p] if op != "pmult" else ys[0]
        assert np.array_equal(host(dst[p]), _want(op, xs[p], y, cx, primes)), p


def test_elementwise_in_place(ctx):
    c, main, aux = ctx
    primes = main[:12]
    r = np.random.default_rng(5)
    x, y = _operand(r, primes), _operand(r, primes)
    dx = dev(x)
    c.elementwise(11, 0, "sub", [dx], [dx], [dev(y)])
    assert np.array_equal(host(dx), _want("sub", x, y, None, primes))


def test_mult_imaginary_unit(ctx):
    c, main, aux = ctx
    level = 23
    primes = main[:level + 1]
    r = np.random.default_rng(6)
    x = _operand(r, primes, edge=True)
    t, u = zeros(len(primes), N), zeros(len(primes), N)
    c.elementwise(level, 0, "mult_i", [t], [dev(x)])
    c.elementwise(level, 0, "mult_i", [u], [t])
    assert np.array_equal(host(u), _want("neg", x, None, None, primes))
    # per limb one factor w with w^2 = -1 on the first half of the NTT
    # points and -w on the second (x[:, 64] = q - 1 is non-zero)
    tx = host(t)
    for i, p in enumerate(primes):
        w = int(tx[i, 64]) * pow(int(x[i, 64]), -1, p) % p
        assert w * w % p == p - 1, i
        half = (x[i].astype(np.uint64) * w % p).astype(np.uint32)
        want = np.concatenate([half[:N // 2], ((p - half[N // 2:].astype(
            np.uint64)) % p).astype(np.uint32)])
        assert np.array_equal(tx[i], want), i
    msg = r.uniform(-1, 1, 1 << 10) + 1j * r.uniform(-1, 1, 1 << 10)
    pt = zeros(len(primes), N)
    c.encode(level, 0, 2.0 ** 30, msg, pt)
    out = zeros(len(primes), N)
    c.elementwise(level, 0, "mult_i", [out], [pt])
    got = c.decode(level, 2.0 ** 30, 1 << 10, out)
    assert np.max(np.abs(got - 1j * msg)) < 1e-3


def test_elementwise_rejects_bad_arguments(ctx):
    import cheddar_amd
    c, main, aux = ctx
    x = zeros(24, N)
    with pytest.raises(cheddar_amd.ChdError):
        c.elementwise(23, 9, "add", [x], [x], [x])         # num_aux > alpha
    with pytest.raises(cheddar_amd.ChdError):
        c.elementwise(23, 0, "add_const", [x], [x])        # no constant
    with pytest.raises(cheddar_amd.ChdError):
        c.elementwise(23, 0, "add", [x] * 4, [x] * 4, [x] * 4)
