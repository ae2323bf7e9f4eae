"""GPU tests of the layers above the hoisted key switch: the min_ks
evaluation order (Hoist.cu:517-566) bit-exact against the oracle's
restatement, and LinearTransform (LinearTransform.cpp) end to end: an
encrypted vector times a matrix given by its diagonals, decrypted on the
host and decoded, against numpy within the reference's 1e-3."""
import numpy as np
import pytest

import _orc
from gpu_util import N, config4, dev, host, uniform_limbs, zeros

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("no HIP device visible")
    import cheddar_amd
    main, aux, levels = config4()
    return cheddar_amd.Context(cheddar_amd.Param(main, aux, levels))


def _rand_keys(r, primes, rots, beta=3):
    return {rot: (np.stack([uniform_limbs(r, primes) for _ in range(beta)]),
                  np.stack([uniform_limbs(r, primes) for _ in range(beta)]))
            for rot in rots}


def _dkeys(keys):
    return {k: ([dev(x) for x in v[0]], [dev(x) for x in v[1]])
            for k, v in keys.items()}


def test_hoist_min_ks_matches_oracle(ctx):
    import cheddar_amd
    import hoist_ref
    main, aux = ctx.param.main, ctx.param.aux
    L = 20
    r = np.random.default_rng(800)
    bsi, gsi = [0, 1, 2, 3], [0, 4, 8]
    pts = {(g, b): uniform_limbs(r, main[:L] + aux) for g in gsi for b in bsi
           if (g, b) != (4, 2)}
    keys = _rand_keys(r, main + aux, [1, 4])
    b_, a_ = uniform_limbs(r, main[:L]), uniform_limbs(r, main[:L])
    wb, wa = hoist_ref.evaluate_min_ks(b_, a_, pts, keys, L, 24, main, aux, 16)
    print("min_ks hoist bs", bsi, "gs", gsi, flush=True)
    h = cheddar_amd.Hoist(ctx, L - 1, gsi, bsi, {k: dev(v) for k, v in
                                                 pts.items()})
    assert h.required_rotations(min_ks=True) == [1, 4]
    assert h.required_rotations() == [1, 2, 3, 4, 8]
    out = (zeros(L - 1, N), zeros(L - 1, N))
    h.run(out, (dev(b_), dev(a_)), _dkeys(keys), min_ks=True)
    assert np.array_equal(host(out[0]), wb)
    assert np.array_equal(host(out[1]), wa)


def test_hoist_min_ks_rejects_incomplete_sequence(ctx):
    import cheddar_amd
    main, aux = ctx.param.main, ctx.param.aux
    L = 20
    r = np.random.default_rng(810)
    pts = {(0, b): dev(uniform_limbs(r, main[:L] + aux)) for b in (0, 1, 3)}
    h = cheddar_amd.Hoist(ctx, L - 1, [0], [0, 1, 3], pts)
    with pytest.raises(cheddar_amd.ChdError, match="MinKS"):
        h.required_rotations(min_ks=True)


def _encrypt(keys, ctx, level, scale, msg):
    L = ctx.param.num_q(level)
    q = ctx.param.main[:L]
    pt = zeros(L, N)
    ctx.encode(level, 0, scale, msg, pt)
    a = keys.uniform(q)
    b = keys._add(keys._add(keys._neg(keys._mul(a, keys.s_ntt[:L], q), q),
                            host(pt), q), keys.ntt_of(keys.small(), q), q)
    return b, a


def _decrypt_decode(keys, ctx, level, scale, slots, res):
    L = ctx.param.num_q(level)
    q = ctx.param.main[:L]
    v = keys._add(host(res[0]), keys._mul(host(res[1]), keys.s_ntt[:L], q), q)
    return ctx.decode(level, scale, slots, dev(v))


@pytest.mark.parametrize("min_ks", [False, True])
def test_linear_transform_decrypts_to_matrix_product(ctx, min_ks):
    """a 256 x 256 matrix with 16 diagonals, bs = gs = 4 (giant steps 0, 4,
    8, 12), on a 256-slot encoding of x"""
    import cheddar_amd
    import ckks_host as ck
    main, aux = ctx.param.main, ctx.param.aux
    level = 19
    dim = 256
    delta = 2.0 ** 30
    pt_scale = float(main[level])
    r = np.random.default_rng(820 + int(min_ks))
    diags = {i: r.uniform(-1, 1, dim) + 1j * r.uniform(-1, 1, dim)
             for i in range(16)}
    x = r.uniform(-1, 1, dim) + 1j * r.uniform(-1, 1, dim)
    y = sum(d * np.roll(x, -i) for i, d in diags.items())
    print("linear transform min_ks", min_ks, flush=True)
    lt = cheddar_amd.Hoist.linear_transform(ctx, level, pt_scale, dim, diags,
                                            bs=4, gs=4)
    rots = lt.required_rotations(min_ks)
    assert rots == ([1, 4] if min_ks else [1, 2, 3, 4, 8, 12])
    keys = ck.Keys(16, main, aux, seed=21)
    rk = {rot: keys.rot_key(_orc.lib.orc_galois_factor(rot, 16), 24)
          for rot in rots}
    b, a = _encrypt(keys, ctx, level, delta, x)
    out = (zeros(level, N), zeros(level, N))
    lt.run(out, (dev(b), dev(a)), _dkeys(rk), min_ks=min_ks)
    got = _decrypt_decode(keys, ctx, level - 1,
                          delta * pt_scale / main[level], dim, out)
    err = np.max(np.abs(got - y))
    print("linear transform max error", err, flush=True)
    assert err < 1e-3
