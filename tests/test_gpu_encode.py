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


# ------------------------------------ hoisting from messages (Hoist.cu) ----
def _rand_keys(r, main, aux, rots, beta=3):
    from gpu_util import uniform_limbs
    primes = main + aux
    out = {}
    for rot in rots:
        kb = np.stack([uniform_limbs(r, primes) for _ in range(beta)])
        ka = np.stack([uniform_limbs(r, primes) for _ in range(beta)])
        out[rot] = (kb, ka)
    return out


def _dkeys(keys):
    from gpu_util import dev
    return {k: ([dev(x) for x in v[0]], [dev(x) for x in v[1]])
            for k, v in keys.items()}


def _encode_ext(ctx, level, scale, msg):
    """oracle plaintext at (level, alpha aux primes)"""
    return _oracle_encode(ctx, level, ctx.param.alpha, scale, msg)[0]


def test_hoist_from_messages_swapped_matches_oracle(ctx):
    """single giant step 0: the reference swaps baby and giant steps and
    rotates each message right by its baby step (Hoist.cu:153-168), then
    takes the bs == 1 path (Hoist.cu:715-797)"""
    import cheddar_amd
    import hoist_ref
    from gpu_util import dev, uniform_limbs
    main, aux = ctx.param.main, ctx.param.aux
    L, level, scale = 20, 19, 2.0 ** 30
    r = np.random.default_rng(700)
    bsi = [0, 1, 2, 5]
    msgs = {(0, b): _msg(710 + b, 1 << 15) for b in bsi}
    keys = _rand_keys(r, main, aux, [b for b in bsi if b])
    b_, a_ = uniform_limbs(r, main[:L]), uniform_limbs(r, main[:L])
    pts = {}
    for b in bsi:
        m = msgs[(0, b)]
        pts[b] = _encode_ext(ctx, level, scale, np.roll(m, b))
    wb, wa = hoist_ref.evaluate_gs_only(b_, a_, pts, keys, L, 24, main, aux, 16)
    print("hoist from messages, swapped, bs", bsi, flush=True)
    h = cheddar_amd.Hoist.from_messages(ctx, level, scale, [0], bsi, msgs)
    out = (zeros(L - 1, 1 << 16), zeros(L - 1, 1 << 16))
    h.run(out, (dev(b_), dev(a_)), _dkeys(keys))
    assert np.array_equal(host(out[0]), wb)
    assert np.array_equal(host(out[1]), wa)


def test_hoist_from_messages_bsgs_matches_oracle(ctx):
    """two giant steps: no swap, plaintexts encoded as given; one absent"""
    import cheddar_amd
    import hoist_ref
    from gpu_util import dev, uniform_limbs
    main, aux = ctx.param.main, ctx.param.aux
    L, level, scale = 20, 19, 2.0 ** 30
    r = np.random.default_rng(720)
    bsi, gsi = [0, 1, 2], [0, 3]
    msgs = {(g, b): _msg(730 + 3 * g + b, 1 << 14) for g in gsi for b in bsi
            if (g, b) != (3, 1)}
    keys = _rand_keys(r, main, aux, [1, 2, 3])
    b_, a_ = uniform_limbs(r, main[:L]), uniform_limbs(r, main[:L])
    pts = {k: _encode_ext(ctx, level, scale, m) for k, m in msgs.items()}
    wb, wa = hoist_ref.evaluate(b_, a_, pts, keys, L, 24, main, aux, 16)
    print("hoist from messages, bsgs", flush=True)
    h = cheddar_amd.Hoist.from_messages(ctx, level, scale, gsi, bsi, msgs)
    out = (zeros(L - 1, 1 << 16), zeros(L - 1, 1 << 16))
    h.run(out, (dev(b_), dev(a_)), _dkeys(keys))
    assert np.array_equal(host(out[0]), wb)
    assert np.array_equal(host(out[1]), wa)


def test_linear_transform_decrypts_to_matrix_product(ctx):
    """end to end: encode x, encrypt under a known secret (host), evaluate a
    banded matrix W through the hoisted handler built from W's diagonals,
    decrypt (host) and decode: W x within the reference's 1e-3
    (Testbed.h:93)"""
    import cheddar_amd
    import ckks_host as ck
    from gpu_util import dev
    main, aux = ctx.param.main, ctx.param.aux
    L, level = 20, 19
    n, s = 1 << 16, 1 << 15
    delta = 2.0 ** 30
    pt_scale = float(main[L - 1])  # result keeps the input scale
    keys = ck.Keys(16, main, aux, seed=11)
    r = np.random.default_rng(740)
    bsi = [0, 1, 2, 3]
    x = _msg(741, s)
    diags = {b: r.uniform(-1, 1, s) + 1j * r.uniform(-1, 1, s) for b in bsi}
    y = sum(diags[b] * np.roll(x, -b) for b in bsi)
    # encryption of Encode(x): b = -a s + pt + e
    q = main[:L]
    pt = zeros(L, n)
    ctx.encode(level, 0, delta, x, pt)
    a_ = keys.uniform(q)
    e = keys.ntt_of(keys.small(), q)
    b_ = keys._add(keys._add(keys._neg(keys._mul(a_, keys.s_ntt[:L], q), q),
                             host(pt), q), e, q)
    rk = {}
    for b in bsi[1:]:
        g = _orc.lib.orc_galois_factor(b, 16)
        rk[b] = keys.rot_key(g, 24)
    print("linear transform: keys ready", flush=True)
    h = cheddar_amd.Hoist.from_messages(ctx, level, pt_scale, [0], bsi,
                                        {(0, b): diags[b] for b in bsi})
    out = (zeros(L - 1, n), zeros(L - 1, n))
    h.run(out, (dev(b_), dev(a_)), _dkeys(rk))
    q1 = main[:L - 1]
    v = keys._add(host(out[0]), keys._mul(host(out[1]), keys.s_ntt[:L - 1],
                                          q1), q1)
    got = ctx.decode(level - 1, delta * pt_scale / main[L - 1], s, dev(v))
    err = np.max(np.abs(got - y))
    print("linear transform max error", err, flush=True)
    assert err < 1e-3
