"""GPU parity at the reference's own parameter files (tests/golden/params/
bootparam_30.json, bootparam_35.json and bootparam_40.json, copied from the
reference's parameters/; the last two have terminal primes): the HIP key
switch through the C-ABI against the oracle compositions of tests/ks_ref.py,
bit-exact, at the real sizes (N = 2^16, up to 48 q limbs, alpha = 12).

The levels cover: the top level; levels missing terminal primes, whose dnum
groups start part-way into the first chain group; rescales that drop
terminal primes and restore main primes and the reverse (the BitPacker
restore and padding); two-prime rescales and 20-bit primes
(bootparam_30); and the encoder at a level made mostly of terminal primes.
"""
import json
import os

import numpy as np
import pytest

import _orc
import ckks_encode as E
from gpu_util import N, dev, host, zeros
from ks_ref import Chain

pytestmark = pytest.mark.gpu

PARAMS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "params")


@pytest.fixture(scope="module", params=["bootparam_30.json",
                                        "bootparam_35.json",
                                        "bootparam_40.json"])
def setup(request):
    import torch
    if not torch.cuda.is_available():
        pytest.fail("no HIP device visible")
    import cheddar_amd
    _orc.lib.orc_set_threads(16)
    text = open(os.path.join(PARAMS, request.param)).read()
    d = json.loads(text)
    param = cheddar_amd.Param.from_json(text)
    ctx = cheddar_amd.Context(param)
    chain = Chain(d["main_primes"], d["terminal_primes"],
                  d["auxiliary_primes"], d["level_config"], 16)
    r = np.random.default_rng(1000 + len(d["terminal_primes"]))
    beta = (chain.max_q + chain.alpha - 1) // chain.alpha
    kp = chain.chain + chain.aux
    kb = np.stack([_uniform(r, kp) for _ in range(beta)])
    ka = np.stack([_uniform(r, kp) for _ in range(beta)])
    dk = ([dev(x) for x in kb], [dev(x) for x in ka])
    print("parameter set", request.param, "levels", len(chain.levels),
          flush=True)
    return request.param, ctx, chain, (kb, ka), dk, r


def _uniform(r, primes):
    return np.stack([r.integers(0, p, N, dtype=np.uint64).astype(np.uint32)
                     for p in primes])


def _levels(chain):
    """a spread of levels: the top two, and the highest and lowest level of
    each restoring rescale (terminal primes leave and main primes return,
    and the reverse)"""
    top = len(chain.levels) - 1
    ter_out, main_out = [], []
    for lv in range(1, top + 1):
        (m, t), (m2, t2) = chain.np(lv), chain.np(lv - 1)
        if t > t2 and m2 > m:
            ter_out.append(lv)
        if m > m2 and t2 > t:
            main_out.append(lv)
    picks = {top, top - 1}
    for lst in (ter_out, main_out):
        if lst:
            picks.update((lst[0], lst[-1]))
    return sorted(picks)


def chain_top(chain):
    return len(chain.levels) - 1


def test_rescale_chain_every_level(setup):
    name, ctx, chain, _, _, r = setup
    top = len(chain.levels) - 1
    b = _uniform(r, chain.q(top))
    a = _uniform(r, chain.q(top))
    for level in range(top, 0, -1):
        nl = len(chain.q(level - 1))
        out = (zeros(nl, N), zeros(nl, N))
        print(name, "rescale level", level, chain.np(level), "->",
              chain.np(level - 1), flush=True)
        ctx.rescale(level, out, (dev(b), dev(a)))
        wb, wa = chain.rescale(b, level), chain.rescale(a, level)
        assert np.array_equal(host(out[0]), wb), (name, level)
        assert np.array_equal(host(out[1]), wa), (name, level)
        b, a = wb, wa


def test_hmult_at_terminal_levels(setup):
    name, ctx, chain, (kb, ka), (dkb, dka), r = setup
    for level in _levels(chain):
        q = chain.q(level)
        b1, a1, b2, a2 = (_uniform(r, q) for _ in range(4))
        for rescale in ((True, False) if level == chain_top(chain)
                        else (True,)):
            nl = len(chain.q(level - 1)) if rescale else len(q)
            out = (zeros(nl, N), zeros(nl, N))
            print(name, "hmult level", level, chain.np(level), "rescale",
                  rescale, flush=True)
            ctx.hmult(level, out, (dev(b1), dev(a1)), (dev(b2), dev(a2)),
                      dkb, dka, rescale=rescale)
            wb, wa = chain.hmult(b1, a1, b2, a2, kb, ka, level, int(rescale))
            assert np.array_equal(host(out[0]), wb), (name, level, rescale)
            assert np.array_equal(host(out[1]), wa), (name, level, rescale)


def test_hrot_and_mod_up_at_offset_levels(setup):
    name, ctx, chain, (kb, ka), (dkb, dka), r = setup
    offset_levels = [lv for lv in range(1, len(chain.levels))
                     if chain.offset(lv) % chain.alpha][-2:] or [
                         len(chain.levels) - 1]
    for level in offset_levels:
        q = chain.q(level)
        b, a = _uniform(r, q), _uniform(r, q)
        out = (zeros(len(q), N), zeros(len(q), N))
        print(name, "hrot level", level, chain.np(level), flush=True)
        ctx.hrot(level, out, (dev(b), dev(a)), dkb, dka, 7)
        wb, wa = chain.hrot(b, a, kb, ka, level, 7)
        assert np.array_equal(host(out[0]), wb), (name, level)
        assert np.array_equal(host(out[1]), wa), (name, level)
        # ModUp: non-empty groups against the oracle
        beta = ctx.beta(level)
        groups = chain.groups(level)
        dst = [zeros(len(q) + chain.alpha, N) for _ in range(beta)]
        ctx.mod_up(level, dst, dev(a))
        want = _orc.mod_up_ex(a, q, chain.aux, chain.offset(level), 16)
        for g in groups:
            assert np.array_equal(host(dst[g]), want[g]), (name, level, g)


def test_mult_key_no_mod_down_at_offset_levels(setup):
    """Context::MultKeyNoModDown through the C-ABI, both forms
    (Context.cpp:609-712): the MultKey branch (ModUp of ax, P * bx), the
    relinearisation branch (ModUp of rx, P * (bx, ax)) and the PAccum of a
    caller-held ModUp, at the top level and at a level whose dnum groups
    start part-way into a chain group (terminal primes missing)"""
    name, ctx, chain, (kb, ka), (dkb, dka), r = setup
    top = chain_top(chain)
    shifted = [lv for lv in range(1, top + 1)
               if chain.offset(lv) % chain.alpha]
    for level in sorted({top} | set(shifted[-1:])):
        q = chain.q(level)
        t = len(q) + chain.alpha
        b, a, rx = (_uniform(r, q) for _ in range(3))
        acc = (zeros(t, N), zeros(t, N))
        print(name, "mult_key_no_mod_down level", level, chain.np(level),
              flush=True)
        ctx.mult_key_no_mod_down(level, acc, (dev(b), dev(a)), dkb, dka)
        wb, wa = chain.key_mult(a, level, kb, ka)
        assert np.array_equal(host(acc[0]), chain.caccum(wb, b, level)), (
            name, level)
        assert np.array_equal(host(acc[1]), wa), (name, level)
        ctx.mult_key_no_mod_down(level, acc, (dev(b), dev(a), dev(rx)), dkb,
                                 dka)
        wb, wa = chain.key_mult(rx, level, kb, ka)
        assert np.array_equal(host(acc[0]), chain.caccum(wb, b, level)), (
            name, level, "rx")
        assert np.array_equal(host(acc[1]), chain.caccum(wa, a, level)), (
            name, level, "rx")
        groups = chain.groups(level)
        up = [zeros(t, N) if g in groups else None
              for g in range(ctx.beta(level))]
        ctx.mod_up(level, up, dev(rx))
        ctx.mult_key_no_mod_down_mod_up(level, acc, up, dkb, dka)
        assert np.array_equal(host(acc[0]), wb), (name, level, "modup")
        assert np.array_equal(host(acc[1]), wa), (name, level, "modup")


def test_encode_decode_at_terminal_level(setup):
    name, ctx, chain, _, _, r = setup
    level = next((lv for lv in range(len(chain.levels))
                  if chain.np(lv)[1] >= 3), len(chain.levels) // 2)
    q = chain.q(level)
    msg = r.uniform(-1, 1, 1 << 12) + 1j * r.uniform(-1, 1, 1 << 12)
    scale = 2.0 ** 30
    for num_aux in (0, chain.alpha):
        primes = q + chain.aux[:num_aux]
        dst = zeros(len(primes), N)
        print(name, "encode level", level, chain.np(level), "aux", num_aux,
              flush=True)
        ctx.encode(level, num_aux, scale, msg, dst)
        mx, _ = E.coefficient_residues(msg.real, msg.imag, primes, 16, scale)
        want = _orc.ntt_batch(mx.reshape(-1), 16, primes, mont=1).reshape(
            len(primes), -1)
        assert np.array_equal(host(dst), want), (name, level, num_aux)
    pt = zeros(len(q), N)
    ctx.encode(level, 0, scale, msg, pt)
    got = ctx.decode(level, scale, 1 << 12, pt)
    assert np.max(np.abs(got - msg)) < 1e-3
