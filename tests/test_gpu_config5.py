"""Config 5 at its real shape: an encrypted BERT-base linear-layer slice.

A 768 x 768 weight W ~ N(0, 0.02) times a 768-wide activation x ~ N(0, 1)
replicated over 2^15 slots, by the BSGS diagonal method with 28 baby steps
(0..27) and 28 giant steps (28 k), at L = 20 limbs of the config-4 chain
(N = 2^16, 24 main primes, 8 aux primes, dnum 3), double hoisting:
  y = sum_g Rot_g(sum_b pt[g][b] * Rot_b(x)),  pt[g][b] = Rot_{-g}(diag_{g+b})
with diag_d[j] = W[j][(j + d) mod 768] on slots j < 768 (768 plaintexts,
54 rotation keys, each giant step a full key switch).

The plaintexts go through the reference's message constructor
(HoistHandler, Hoist.cu:131-177) and the evaluation through the handle
(EvaluateGiantStepOptimized, Hoist.cu:840-975; GSFusedKernel,
Hoist.cu:80-118), which at this shape runs the wide giant-step
accumulation over 28 giant steps and the batched giant-step key switches.

- bit-exact: the result residues against the oracle's restatement of the
  same evaluation (tests/hoist_ref.py) on the same ciphertext, keys and
  plaintext residues (host coefficient residues, pinned against the numpy
  restatement of the encoder on a sample here and in test_encode.py, then
  the oracle's NTT with Montgomery conversion);
- semantic: the decrypted, decoded result against numpy W x within the
  reference's 1e-3 (Testbed.h:93), zero beyond the 768 output slots.
"""
import os
import sys
from collections.abc import Mapping

import numpy as np
import pytest

import _orc
from gpu_util import N, config4, dev, host, zeros

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]

DIM = 768
BS = list(range(28))
GS = [28 * k for k in range(28)]
LEVEL = 19            # L = 20 q limbs
SLOTS = 1 << 15
DELTA = 2.0 ** 30     # activation scale
PT_SCALE = 2.0 ** 30  # weight scale


def _progress(msg):
    # set-up phases take tens of seconds: report them as they finish
    print("config5: " + msg, file=sys.__stdout__, flush=True)


def _workers():
    return max(1, min(16, os.cpu_count() or 1))


def _message(W, g, b):
    """Rot_{-g}(diag_{g+b}) over 2^15 slots"""
    rows = np.arange(DIM)
    diag = np.zeros(SLOTS)
    diag[:DIM] = W[rows, (rows + g + b) % DIM]
    return np.roll(diag, g).astype(np.complex128)


def _pairs():
    return [(g, b) for g in GS for b in BS if g + b < DIM]


class _Plaintexts(Mapping):
    """(g, b) -> the oracle's plaintext, computed when read, into one reused
    buffer: host coefficient residues (pinned against the numpy
    restatement on a sample in the test), then the oracle's NTT with
    Montgomery conversion"""

    def __init__(self, param, W, primes):
        self.param, self.W = param, W
        self.primes = _orc.u32(primes)
        self.keys = set(_pairs())
        self.buf = np.empty((len(primes), N), np.uint32)

    def __getitem__(self, key):
        if key not in self.keys:
            raise KeyError(key)
        _, slots = self.param.encode_coefficients(
            LEVEL, len(self.primes) - LEVEL - 1, PT_SCALE,
            _message(self.W, *key), out=self.buf)
        assert slots == SLOTS
        _orc.lib.orc_ntt_batch(self.buf, len(self.primes), 16, self.primes,
                               1)
        return self.buf

    def __contains__(self, key):
        return key in self.keys

    def __iter__(self):
        return iter(sorted(self.keys))

    def __len__(self):
        return len(self.keys)


class _HostKeys(Mapping):
    """rot -> (key_b, key_a) copied from the device keys the GPU ran with,
    into reused host buffers"""

    def __init__(self, dkeys):
        self.dkeys = dkeys
        self.rot = None
        kb0 = dkeys[next(iter(dkeys))][0]
        shape = (len(kb0),) + tuple(kb0[0].shape)
        self.kb = np.empty(shape, np.uint32)
        self.ka = np.empty(shape, np.uint32)

    def __getitem__(self, rot):
        if rot not in self.dkeys:
            raise KeyError(rot)
        if rot != self.rot:
            import torch
            for buf, parts in ((self.kb, self.dkeys[rot][0]),
                               (self.ka, self.dkeys[rot][1])):
                for g, t in enumerate(parts):
                    torch.from_numpy(buf[g].view(np.int32)).copy_(t)
            self.rot = rot
        return self.kb, self.ka

    def __contains__(self, rot):
        return rot in self.dkeys

    def __iter__(self):
        return iter(sorted(self.dkeys))

    def __len__(self):
        return len(self.dkeys)


@pytest.fixture(scope="module")
def cfg5():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("no HIP device visible")
    import cheddar_amd
    import ckks_host as ck
    main, aux, levels = config4()
    param = cheddar_amd.Param(main, aux, levels)
    ctx = cheddar_amd.Context(param)
    _orc.lib.orc_set_threads(_workers())
    r = np.random.default_rng(0xC0FFEE05)
    W = r.normal(0.0, 0.02, (DIM, DIM))
    x = r.normal(0.0, 1.0, DIM)

    # 54 real rotation keys (s(X^(g^-1)) -> s), each drawn from its own
    # seed and kept on the device only
    keys = ck.Keys(16, main, aux, seed=0x5EED)
    rots = sorted(set(BS[1:] + GS[1:]))
    assert len(rots) == 54
    dkeys = {}
    for rot in rots:
        kb, ka = keys.rot_key(_orc.lib.orc_galois_factor(rot, 16), 24,
                              rng=np.random.default_rng([0x5EED, rot]))
        dkeys[rot] = ([dev(t) for t in kb], [dev(t) for t in ka])
    _progress("54 rotation keys generated")

    # encrypt x replicated over the slots (b = -a s + m + e)
    L = LEVEL + 1
    q = main[:L]
    pt = zeros(L, N)
    ctx.encode(LEVEL, 0, DELTA, np.resize(x, SLOTS).astype(np.complex128),
               pt)
    a = keys.uniform(q)
    b = keys._add(keys._add(keys._neg(keys._mul(a, keys.s_ntt[:L], q), q),
                            host(pt), q), keys.ntt_of(keys.small(), q), q)
    del pt

    msgs = {k: _message(W, *k) for k in _pairs()}
    assert len(msgs) == DIM
    h = cheddar_amd.Hoist.from_messages(ctx, LEVEL, PT_SCALE, GS, BS, msgs)
    del msgs
    h._keep = None
    assert h.required_rotations() == rots
    _progress("handle built (768 plaintexts encoded by the library)")
    return dict(ctx=ctx, param=param, main=main, aux=aux, W=W, x=x,
                keys=keys, dkeys=dkeys, ct=(b, a), h=h)


def _run(c):
    out = (zeros(LEVEL, N), zeros(LEVEL, N))
    c["h"].run(out, (dev(c["ct"][0]), dev(c["ct"][1])), c["dkeys"])
    return host(out[0]), host(out[1])


def test_config5_residues_match_oracle(cfg5):
    import ckks_encode as E
    import hoist_ref
    c = cfg5
    main, aux = c["main"], c["aux"]
    primes = main[:LEVEL + 1] + aux
    # the encoder's host half at this shape against the numpy restatement,
    # on a sample of diagonals (first, last, and of different giant steps)
    for key in [(0, 0), (28, 5), (392, 27), (756, 11)]:
        msg = _message(c["W"], *key)
        got, _ = c["param"].encode_coefficients(LEVEL, len(aux), PT_SCALE,
                                                msg)
        want, _ = E.coefficient_residues(msg.real, msg.imag, primes, 16,
                                         PT_SCALE)
        assert np.array_equal(got, np.asarray(want).reshape(got.shape)), key
    got_b, got_a = _run(c)
    _progress("GPU evaluation done")
    want_b, want_a = hoist_ref.evaluate(
        c["ct"][0], c["ct"][1], _Plaintexts(c["param"], c["W"], primes),
        _HostKeys(c["dkeys"]), LEVEL + 1, 24, main, aux, 16)
    _progress("oracle evaluation done")
    assert np.array_equal(got_b, want_b)
    assert np.array_equal(got_a, want_a)


def test_config5_decrypts_to_matrix_product(cfg5):
    c = cfg5
    main = c["main"]
    got_b, got_a = _run(c)
    keys = c["keys"]
    q = main[:LEVEL]
    v = keys._add(got_b, keys._mul(got_a, keys.s_ntt[:LEVEL], q), q)
    scale = DELTA * PT_SCALE / main[LEVEL]
    y = c["ctx"].decode(LEVEL - 1, scale, SLOTS, dev(v))
    want = c["W"] @ c["x"]
    err = np.max(np.abs(y[:DIM] - want))
    tail = np.max(np.abs(y[DIM:]))
    _progress("max error %.3g, beyond 768 slots %.3g" % (err, tail))
    assert err < 1e-3
    assert tail < 1e-3
