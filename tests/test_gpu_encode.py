"""GPU parity of the encoder entry points (chd_encode, chd_decode,
chd_encode_constant) against the CPU oracle (oracle/ckks_encode.py plus the
C oracle's NTT), bit-exact, at the config-4 parameters (N = 2^16, 24 q
primes, 8 aux primes); plus the reference's own EncodeDecode check
(unittest/BasicTest.cpp:10-25: decode(encode(m)) within 1e-3)."""
import numpy as np
import pytest

import _orc
import ckks_encode as E
from gpu_util import config4, host, zeros

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("no HIP device visible")
    import cheddar_amd
    main, aux, levels = config4()
    param = cheddar_amd.Param(main, aux, levels)
    return cheddar_amd.Context(param)


def _msg(seed, n):
    r = np.random.default_rng(seed)
    return r.uniform(-1, 1, n) + 1j * r.uniform(-1, 1, n)


def _primes(ctx, level, num_aux):
    p = ctx.param
    return p.main[:p.num_q(level)] + p.aux[:num_aux]


def _oracle_encode(ctx, level, num_aux, scale, msg):
    primes = _primes(ctx, level, num_aux)
    mx, slots = E.coefficient_residues(msg.real, msg.imag, primes, 16, scale)
    return _orc.ntt_batch(mx.reshape(-1), 16, primes, mont=1).reshape(
        len(primes), -1), slots


def _oracle_decode(primes, pt, slots, scale):
    icrt = E.icrt_constants(primes, 1 << 16)
    scaled = np.stack([
        _orc.intt_mult_const(pt[i], 16, q, icrt[i], 0).view(np.uint32)
        for i, q in enumerate(primes)])
    return E.decode_values(scaled, primes, 16, slots, scale)


@pytest.mark.parametrize("level,num_aux,length", [
    (23, 0, 1 << 15), (19, 8, 1 << 15), (0, 0, 3), (9, 8, 1000)])
def test_encode_matches_oracle(ctx, level, num_aux, length):
    scale = 2.0 ** 30
    msg = _msg(level * 7 + length, length)
    limbs = ctx.param.num_q(level) + num_aux
    dst = zeros(limbs, 1 << 16)
    print("encode level", level, "aux", num_aux, "len", length, flush=True)
    slots = ctx.encode(level, num_aux, scale, msg, dst)
    want, wslots = _oracle_encode(ctx, level, num_aux, scale, msg)
    assert slots == wslots
    assert np.array_equal(host(dst), want)


@pytest.mark.parametrize("level,length", [(23, 1 << 15), (4, 1 << 12)])
def test_decode_matches_oracle_and_round_trips(ctx, level, length):
    scale = 2.0 ** 30
    msg = _msg(50 + level, length)
    dst = zeros(ctx.param.num_q(level), 1 << 16)
    print("decode level", level, "len", length, flush=True)
    slots = ctx.encode(level, 0, scale, msg, dst)
    got = ctx.decode(level, scale, slots, dst)
    # the reference's EncodeDecode tolerance (Testbed.h:93)
    assert np.max(np.abs(got - msg)) < 1e-3
    pt = host(dst)
    wr, wi = _oracle_decode(_primes(ctx, level, 0), pt, slots, scale)
    assert np.array_equal(got.real, wr) and np.array_equal(got.imag, wi)


def test_encode_constant_matches_oracle(ctx):
    for level, num_aux, number, scale in ((23, 0, 0.3, 2.0 ** 30),
                                          (10, 8, -2.5, 2.0 ** 40),
                                          (0, 0, 1.0, 2.0 ** 70)):
        dst = zeros(ctx.param.num_q(level) + num_aux)
        ctx.encode_constant(level, num_aux, scale, number, dst)
        want = E.encode_constant(number, _primes(ctx, level, num_aux), scale)
        assert np.array_equal(host(dst), want)


def test_encode_rejects_invalid(ctx):
    import cheddar_amd
    dst = zeros(24, 1 << 16)
    with pytest.raises(cheddar_amd.ChdError):
        ctx.encode(23, 3, 2.0 ** 30, _msg(1, 8), dst)        # aux not alpha
    with pytest.raises(cheddar_amd.ChdError):
        ctx.decode(23, 2.0 ** 30, 3, dst)                      # 3 slots
