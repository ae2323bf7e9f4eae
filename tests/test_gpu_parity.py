"""GPU parity: the HIP path through the C-ABI against the CPU oracle,
bit-exact, on seeded inputs at the BASELINE configurations' real sizes."""
import ctypes

import numpy as np
import pytest

import _orc
from gpu_util import (CFG1_Q, N, Q30, Q31, centred_limbs, config4, dev, host,
                      uniform_limbs, zeros)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def chd():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("no HIP device visible")
    import cheddar_amd
    return cheddar_amd


def rng(s):
    return np.random.default_rng(s)


# ------------------------------------------------------------------ NTT ----
def test_ntt_config1_single_limb_roundtrip(chd):
    plan = chd.NttPlan([CFG1_Q])
    x = uniform_limbs(rng(1), [CFG1_Q])
    src = dev(x)
    y = zeros(N)
    for mont in (0, 1):
        plan.forward(y, src, 1, 1, mont_conv=mont)
        assert np.array_equal(host(y), _orc.ntt(x[0], 16, CFG1_Q, mont))
        back = zeros(N)
        plan.inverse(back, y, 1, 1, mont_conv=mont)
        assert np.array_equal(host(back), x[0])


def test_ntt_config2_batch(chd):
    primes = Q30[:32]
    plan = chd.NttPlan(primes)
    x = np.stack([uniform_limbs(rng(10 + p), primes) for p in range(2)])
    src = dev(x)
    y = zeros(2, 32, N)
    plan.forward(y, src, 32, 2)
    want = np.stack([_orc.ntt_batch(x[p].reshape(-1), 16, primes).reshape(
        32, N) for p in range(2)])
    assert np.array_equal(host(y), want)
    z = zeros(2, 32, N)
    plan.inverse(z, y, 32, 2, mont_conv=True)
    want_inv = np.stack([_orc.intt_batch(want[p].reshape(-1), 16, primes,
                                         1).reshape(32, N) for p in range(2)])
    assert np.array_equal(host(z), want_inv)
    plan.inverse(z, y, 32, 2, mont_conv=False)
    assert np.array_equal(host(z), x)
    # Montgomery conversion on input: out of place (single-pass kernel,
    # constant folded into its first stages) and in place (two passes)
    want_m = np.stack([_orc.ntt_batch(x[p].reshape(-1), 16, primes, 1)
                       .reshape(32, N) for p in range(2)])
    plan.forward(y, src, 32, 2, mont_conv=True)
    assert np.array_equal(host(y), want_m)
    y2 = dev(x)
    plan.forward(y2, y2, 32, 2, mont_conv=True)
    assert np.array_equal(host(y2), want_m)


def test_ntt_forward_two_pass_config2(chd):
    """chd_ntt_forward_two_pass (the two-pass kernels at any size) gives the
    default forward's residues at config 2: out of place, in place, and
    with the Montgomery conversion on input"""
    primes = Q30[:32]
    plan = chd.NttPlan(primes)
    x = np.stack([uniform_limbs(rng(15 + p), primes) for p in range(2)])
    src = dev(x)
    want = np.stack([_orc.ntt_batch(x[p].reshape(-1), 16, primes).reshape(
        32, N) for p in range(2)])
    y = zeros(2, 32, N)
    plan.forward(y, src, 32, 2, two_pass=True)
    assert np.array_equal(host(y), want)
    assert np.array_equal(host(src), x)
    want_m = np.stack([_orc.ntt_batch(x[p].reshape(-1), 16, primes, 1)
                       .reshape(32, N) for p in range(2)])
    plan.forward(y, src, 32, 2, mont_conv=True, two_pass=True)
    assert np.array_equal(host(y), want_m)
    y2 = dev(x)
    plan.forward(y2, y2, 32, 2, two_pass=True)
    assert np.array_equal(host(y2), want)


@pytest.mark.parametrize("bits", [30, 31])
def test_ntt_inverse_single_pass(chd, bits):
    """the single-pass inverse over residue classes (chd_ntt_inverse_single_
    pass) at the config-2 shape, on 30-bit primes (lazy butterflies) and
    31-bit primes (reference-form butterflies), both epilogue constants,
    against the oracle; an overlapping destination is refused"""
    primes = (Q30 if bits == 30 else Q31)[:32]
    plan = chd.NttPlan(primes)
    x = np.stack([uniform_limbs(rng(960 + bits + p), primes)
                  for p in range(2)])
    y = np.stack([_orc.ntt_batch(x[p].reshape(-1), 16, primes).reshape(32, N)
                  for p in range(2)])
    src = dev(y)
    z = zeros(2, 32, N)
    plan.inverse(z, src, 32, 2, mont_conv=False, single_pass=True)
    assert np.array_equal(host(z), x)
    assert np.array_equal(host(src), y)
    want = np.stack([_orc.intt_batch(y[p].reshape(-1), 16, primes,
                                     1).reshape(32, N) for p in range(2)])
    plan.inverse(z, src, 32, 2, mont_conv=True, single_pass=True)
    assert np.array_equal(host(z), want)
    with pytest.raises(chd.ChdError, match="apart from the destination"):
        plan.inverse(src, src, 32, 2, single_pass=True)
    assert np.array_equal(host(src), y)


def test_ntt_31bit_primes_batch(chd):
    """the config-2 batch shape on 31-bit primes (the reference-form
    butterflies of every kernel) against the oracle, both directions"""
    primes = Q31[:32]
    plan = chd.NttPlan(primes)
    x = np.stack([uniform_limbs(rng(950 + p), primes) for p in range(2)])
    y = zeros(2, 32, N)
    plan.forward(y, dev(x), 32, 2)
    want = np.stack([_orc.ntt_batch(x[p].reshape(-1), 16, primes).reshape(
        32, N) for p in range(2)])
    assert np.array_equal(host(y), want)
    z = zeros(2, 32, N)
    plan.inverse(z, y, 32, 2, mont_conv=False)
    assert np.array_equal(host(z), x)
    yi = dev(x)
    plan.forward(yi, yi, 32, 2)          # in place: the two-pass kernels
    assert np.array_equal(host(yi), want)


def test_ntt_concurrent_streams(chd):
    """one plan used from three streams at once on separate buffer sets (the
    benchmark's headline loop): every forward matches the oracle and every
    inverse restores its input"""
    import ctypes
    import torch
    primes = Q30[:32]
    plan = chd.NttPlan(primes)
    sets = 6
    xs = [np.stack([uniform_limbs(rng(900 + 2 * i + p), primes)
                    for p in range(2)]) for i in range(sets)]
    srcs = [dev(x) for x in xs]
    fwds = [zeros(2, 32, N) for _ in range(sets)]
    backs = [zeros(2, 32, N) for _ in range(sets)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in range(3)]
    for rep in range(2):
        for i in range(sets):
            s = ctypes.c_void_p(streams[i % 3].cuda_stream)
            plan.forward(fwds[i], srcs[i], 32, 2, stream=s)
            plan.inverse(backs[i], fwds[i], 32, 2, mont_conv=False, stream=s)
    torch.cuda.synchronize()
    for i in range(sets):
        assert np.array_equal(host(backs[i]), xs[i]), i
    for i in (0, sets - 1):
        want = np.stack([_orc.ntt_batch(xs[i][p].reshape(-1), 16, primes)
                         .reshape(32, N) for p in range(2)])
        assert np.array_equal(host(fwds[i]), want), i


def test_ntt_three_streams_in_place_rounds(chd):
    """the benchmark's headline loop at its size: 33 buffer sets (> 1 GiB,
    more than twice the MALL) rotated over three streams, each step a
    forward into the set's second buffer and the inverse back into its
    source, checked after every round. Under this load a store-data hazard
    once put index values into single words of the forward's output (a
    16-byte buffer store whose data registers were rewritten right after
    it); every forward must equal the first one and every source must come
    back."""
    import ctypes
    import torch
    primes = Q30[:32]
    plan = chd.NttPlan(primes)
    x = np.stack([uniform_limbs(rng(950 + p), primes) for p in range(2)])
    base = dev(x)
    want = zeros(2, 32, N)
    plan.forward(want, base, 32, 2)
    torch.cuda.synchronize()
    sets = 33
    srcs = [base.clone() for _ in range(sets)]
    dsts = [zeros(2, 32, N) for _ in range(sets)]
    streams = [torch.cuda.Stream() for _ in range(3)]
    sps = [ctypes.c_void_p(s.cuda_stream) for s in streams]
    for rnd in range(8):
        for i in range(sets):
            plan.forward(dsts[i], srcs[i], 32, 2, stream=sps[i % 3])
            plan.inverse(srcs[i], dsts[i], 32, 2, mont_conv=False,
                         stream=sps[i % 3])
        torch.cuda.synchronize()
        bad = [i for i in range(sets)
               if not (torch.equal(dsts[i], want) and
                       torch.equal(srcs[i], base))]
        assert not bad, (rnd, bad)


@pytest.mark.parametrize("kind", ["zeros", "max", "impulse", "ramp"])
def test_ntt_edge_inputs(chd, kind):
    primes = [CFG1_Q, Q31[5], Q30[0], Q30[31]]
    if kind == "zeros":
        x = np.zeros((4, N), np.uint32)
    elif kind == "max":
        x = np.stack([np.full(N, p - 1, np.uint32) for p in primes])
    elif kind == "impulse":
        x = np.zeros((4, N), np.uint32)
        x[:, 1] = 1
        x[:, N - 1] = 7
    else:
        x = np.stack([(np.arange(N, dtype=np.uint64) * 2654435761 % p)
                      .astype(np.uint32) for p in primes])
    plan = chd.NttPlan(primes)
    y = zeros(4, N)
    want = _orc.ntt_batch(x.reshape(-1), 16, primes).reshape(4, N)
    plan.forward(y, dev(x), 4, 1)   # single pass (source apart)
    assert np.array_equal(host(y), want)
    yi = dev(x)
    plan.forward(yi, yi, 4, 1)      # in place: two passes
    assert np.array_equal(host(yi), want)
    z = zeros(4, N)
    plan.inverse(z, y, 4, 1, mont_conv=False)
    assert np.array_equal(host(z), x)


# ---------------------------------------------------------------- BConv ----
def test_bconv_config3(chd):
    src_p, dst_p = Q30[:8], Q31[:40]
    plan = chd.BconvPlan(src_p, dst_p)
    c1, c2 = plan.constants()
    o1, o2 = _orc.modswitch_consts(src_p, dst_p, 16)
    assert np.array_equal(c1, o1) and np.array_equal(c2, o2)
    x = centred_limbs(rng(3), src_p)
    out = zeros(40, N)
    plan.apply(out, dev(x.view(np.uint32)))
    assert np.array_equal(host(out), _orc.bconv(x, o2, dst_p, 16))


def test_bconv_extreme_centred_values(chd):
    src_p, dst_p = Q31[:8], Q31[8:20]
    plan = chd.BconvPlan(src_p, dst_p)
    _, o2 = _orc.modswitch_consts(src_p, dst_p, 16)
    x = np.stack([np.where(np.arange(N) % 2 == 0, (p - 1) // 2,
                           -((p - 1) // 2)).astype(np.int32) for p in src_p])
    out = zeros(12, N)
    plan.apply(out, dev(x.view(np.uint32)))
    assert np.array_equal(host(out), _orc.bconv(x, o2, dst_p, 16))


@pytest.mark.parametrize("src_len", [17, 24, 32])
def test_bconv_two_k_chunks(chd, src_len):
    """more than 16 sources take a second MFMA K chunk (ModDownAndRescale of
    five terminal primes plus twelve aux primes needs 17)"""
    src_p, dst_p = (Q30 + Q31)[:src_len], Q31[16:40]
    plan = chd.BconvPlan(src_p, dst_p)
    _, o2 = _orc.modswitch_consts(src_p, dst_p, 16)
    x = centred_limbs(rng(40 + src_len), src_p)
    x[:, :64] = np.array([(p - 1) // 2 for p in src_p], np.int32)[:, None]
    out = zeros(len(dst_p), N)
    plan.apply(out, dev(x.view(np.uint32)))
    assert np.array_equal(host(out), _orc.bconv(x, o2, dst_p, 16))


@pytest.mark.parametrize("src_len,dst_len", [
    (1, 1), (3, 5), (8, 8), (8, 9), (7, 16), (8, 17), (5, 23), (8, 24),
    (8, 25), (9, 24), (16, 8), (16, 24), (2, 40)])
def test_bconv_tile_shapes(chd, src_len, dst_len):
    """full, partial and packed last destination tiles: with at most 8
    sources a last tile of 1..8 destinations carries both coefficient groups
    of a wave in the two K halves; 9 or more sources, or more than 8 in the
    last tile, keep the plain layout"""
    src_p, dst_p = Q30[:src_len], Q31[:dst_len]
    plan = chd.BconvPlan(src_p, dst_p)
    _, o2 = _orc.modswitch_consts(src_p, dst_p, 16)
    x = centred_limbs(rng(100 + 50 * src_len + dst_len), src_p)
    x[:, :32] = np.array([(p - 1) // 2 for p in src_p], np.int32)[:, None]
    x[:, 32:64] = -x[:, :32]
    out = zeros(dst_len, N)
    plan.apply(out, dev(x.view(np.uint32)))
    assert np.array_equal(host(out), _orc.bconv(x, o2, dst_p, 16))


class _Tables(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("q", "qinv", "tw", "itw",
                                               "twist")]


class _LimbMap(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("num_q", "skip_lo", "skip_len",
                                            "src_gap", "tab_off", "tab_gap",
                                            "cst_gap")]


class _BconvJob(ctypes.Structure):
    _fields_ = [("dst", ctypes.c_void_p), ("src", ctypes.c_void_p),
                ("table", ctypes.c_void_p), ("src_len", ctypes.c_int),
                ("dst_len", ctypes.c_int), ("skip_lo", ctypes.c_int),
                ("skip_len", ctypes.c_int)]


# (src_len, dst_len, skip_lo, skip_len) per job: one to three destination
# tiles, packed and plain last tiles, two K chunks, skip ranges before,
# inside and past the destinations
_BATCHES = {
    2: [(8, 24, 8, 8), (8, 23, 0, 0)],
    3: [(8, 24, 0, 8), (8, 24, 8, 8), (5, 27, 16, 5)],
    4: [(17, 40, 0, 0), (32, 9, 3, 2), (8, 16, 0, 0), (1, 5, 2, 30)],
    5: [(8, 24, 0, 8), (8, 24, 8, 8), (17, 40, 0, 0), (5, 27, 16, 5),
        (32, 9, 3, 2)],
    9: [(8, 21, 8, 8)] * 6 + [(9, 33, 1, 1), (16, 8, 0, 0), (2, 17, 20, 4)],
}


@pytest.mark.parametrize("num_jobs", sorted(_BATCHES))
def test_bconv_batch_job_counts(chd, num_jobs):
    """chd_k_bconv_batch (the key switch's entry) against the oracle, each
    job with its own sources, table, lengths and skip range; a batch of two
    to four jobs takes the column-tile workgroup mapping, a larger one the
    consecutive mapping, and both walk every destination tile of a job in
    one workgroup"""
    import torch
    lib = chd.lib
    P = ctypes.c_void_p
    lib.chd_k_bconv_batch.argtypes = [P, P, P, ctypes.c_int, P]
    lib.chd_bconv_table_size.restype = ctypes.c_longlong
    lib.chd_bconv_table_pack.argtypes = [P, P, P, ctypes.c_int, ctypes.c_int]
    dst_q = Q31[:48]
    qinv = np.array([pow(p, -1, 1 << 32) for p in dst_q], np.uint32)
    dq = torch.from_numpy(np.array(dst_q, np.uint32).view(np.int32)).cuda()
    dqi = torch.from_numpy(qinv.view(np.int32)).cuda()
    tabs = _Tables(q=dq.data_ptr(), qinv=dqi.data_ptr())
    lmap = _LimbMap(num_q=1 << 20)
    r = rng(900 + num_jobs)
    jobs, keep, want = (_BconvJob * num_jobs)(), [], []
    for j, (src_len, dst_len, lo, ln) in enumerate(_BATCHES[num_jobs]):
        pos = [k + (ln if k >= lo else 0) for k in range(dst_len)]
        src_p = Q30[:src_len]
        dst_p = [dst_q[p] for p in pos]
        _, t2 = _orc.modswitch_consts(src_p, dst_p, 16)
        x = centred_limbs(r, src_p)
        x[:, :64] = np.array([(p - 1) // 2 for p in src_p], np.int32)[:, None]
        size = lib.chd_bconv_table_size(src_len, dst_len)
        packed = np.zeros(size, np.int8)
        assert lib.chd_bconv_table_pack(
            packed.ctypes.data, np.ascontiguousarray(t2, np.int32).ctypes.data,
            np.array(dst_p, np.uint32).ctypes.data, src_len, dst_len) == 0
        dtab = torch.from_numpy(packed).cuda()
        dsrc = dev(x.view(np.uint32))
        out = zeros(max(pos) + 1, N)
        keep += [dtab, dsrc, out]
        jobs[j] = _BconvJob(out.data_ptr(), dsrc.data_ptr(), dtab.data_ptr(),
                            src_len, dst_len, lo, ln)
        want.append((out, pos, _orc.bconv(x, t2, dst_p, 16)))
    assert lib.chd_k_bconv_batch(ctypes.byref(tabs), ctypes.byref(lmap), jobs,
                                 num_jobs, None) == 0
    torch.cuda.synchronize()
    for j, (out, pos, w) in enumerate(want):
        got = host(out)
        for k, p in enumerate(pos):
            assert np.array_equal(got[p], w[k]), (num_jobs, j, k)


# --------------------------------------------------- key-switch pipeline ----
@pytest.fixture(scope="module")
def ks(chd):
    main, aux, levels = config4(24)
    param = chd.Param(main, aux, levels)
    ctx = chd.Context(param)
    return param, ctx, main, aux


def _evk(r, main, aux, beta):
    primes = main + aux
    kb = np.stack([uniform_limbs(r, primes) for _ in range(beta)])
    ka = np.stack([uniform_limbs(r, primes) for _ in range(beta)])
    return kb, ka


@pytest.mark.parametrize("L,layout", [(24, "strided"), (20, "strided"),
                                      (17, "strided"), (24, "separate"),
                                      (17, "separate")])
def test_mod_up(chd, ks, L, layout):
    """Group outputs equally spaced in one buffer take the batched launch;
    separately allocated ones take the per-group NTT."""
    param, ctx, main, aux = ks
    level = L - 1
    x = uniform_limbs(rng(100 + L), main[:L])
    beta = ctx.beta(level)
    assert beta == (L + 7) // 8
    if layout == "strided":
        whole = zeros(beta * (L + 8), N)
        outs = [whole[g * (L + 8):(g + 1) * (L + 8)] for g in range(beta)]
    else:
        # a gap between the groups rules out the strided path
        whole = zeros(beta * (L + 9), N)
        outs = [whole[g * (L + 9):g * (L + 9) + L + 8] for g in range(beta)]
    ctx.mod_up(level, outs, dev(x))
    want = _orc.mod_up(x, main[:L], aux, 16)
    for g in range(beta):
        assert np.array_equal(host(outs[g]), want[g]), "group %d" % g


@pytest.mark.parametrize("L", [24, 9])
def test_mod_down_family(chd, ks, L):
    param, ctx, main, aux = ks
    level = L - 1
    primes = main[:L] + aux
    x = uniform_limbs(rng(200 + L), primes)
    out = zeros(L, N)
    ctx.mod_down(level, out, dev(x))
    assert np.array_equal(host(out), _orc.mod_down(x, primes, L, 16))
    out2 = zeros(L - 1, N)
    ctx.mod_down_and_rescale(level, out2, dev(x))
    assert np.array_equal(host(out2), _orc.mod_down(x, primes, L - 1, 16))
    xq = np.ascontiguousarray(x[:L])
    out3 = zeros(L - 1, N)
    ctx.rescale_poly(level, out3, dev(xq))
    assert np.array_equal(host(out3), _orc.mod_down(xq, main[:L], L - 1, 16))


def test_tensor(chd, ks):
    param, ctx, main, _ = ks
    L = 24
    r = rng(300)
    b1, a1, b2, a2 = (uniform_limbs(r, main) for _ in range(4))
    res = [zeros(L, N) for _ in range(3)]
    ctx.tensor(L - 1, res, (dev(b1), dev(a1)), (dev(b2), dev(a2)))
    want = _orc.tensor(b1, a1, b2, a2, main, 16)
    for got, w in zip(res, want):
        assert np.array_equal(host(got), w)
    # squaring path (same source pointers)
    sa, sb = dev(a1), dev(b1)
    ctx.tensor(L - 1, res, (sb, sa), (sb, sa))
    want = _orc.tensor(b1, a1, b1, a1, main, 16)
    for got, w in zip(res, want):
        assert np.array_equal(host(got), w)


@pytest.mark.parametrize("L,rescale", [(24, True), (24, False), (20, True)])
def test_hmult_config4(chd, ks, L, rescale):
    param, ctx, main, aux = ks
    level = L - 1
    r = rng(400 + L + int(rescale))
    b1, a1, b2, a2 = (uniform_limbs(r, main[:L]) for _ in range(4))
    kb, ka = _evk(r, main, aux, 3)
    out_l = L - 1 if rescale else L
    res = (zeros(out_l, N), zeros(out_l, N))
    ctx.hmult(level, res, (dev(b1), dev(a1)), (dev(b2), dev(a2)),
              [dev(k) for k in kb], [dev(k) for k in ka], rescale=rescale)
    wb, wa = _orc.hmult(b1, a1, b2, a2, kb, ka, L, 24, main, aux, 16,
                        1 if rescale else 0)
    assert np.array_equal(host(res[0]), wb)
    assert np.array_equal(host(res[1]), wa)


@pytest.mark.parametrize("L,rescale", [(1, False), (2, True), (8, True),
                                       (9, True), (9, False), (16, True),
                                       (17, True)])
def test_hmult_level_sweep(chd, ks, L, rescale):
    """HMult at the low levels of the config-4 chain: one dnum group (L <= 8),
    a partial last group (9, 17), exact multiples (8, 16) and the bottom
    level without rescale, against the oracle"""
    test_hmult_config4(chd, ks, L, rescale)


def test_hmult_in_place_and_separate_rescale(chd, ks):
    param, ctx, main, aux = ks
    L = 24
    r = rng(450)
    b1, a1, b2, a2 = (uniform_limbs(r, main) for _ in range(4))
    kb, ka = _evk(r, main, aux, 3)
    ta, tb = dev(a1), dev(b1)
    ctx.hmult(L - 1, (tb, ta), (tb, ta), (dev(b2), dev(a2)),
              [dev(k) for k in kb], [dev(k) for k in ka], rescale=False)
    wb, wa = _orc.hmult(b1, a1, b2, a2, kb, ka, L, 24, main, aux, 16, 0)
    assert np.array_equal(host(tb), wb) and np.array_equal(host(ta), wa)
    rb, ra = zeros(L - 1, N), zeros(L - 1, N)
    ctx.rescale(L - 1, (rb, ra), (tb, ta))
    assert np.array_equal(host(rb), _orc.rescale(wb, main, L, 1, 16))
    assert np.array_equal(host(ra), _orc.rescale(wa, main, L, 1, 16))


@pytest.mark.parametrize("rescale", [True, False])
def test_hmult_one_aux_prime(chd, rescale):
    """alpha = 1 (dnum = L = 4): ModDown has a single source limb. With so
    few destination limbs (at most 12 polynomial-limbs for one source) the
    one-source BConv writes the destination and the two-pass ModDown NTT
    runs in place on it; without rescale the result is also rescaled
    separately (one source again, the same path), both against the oracle.
    The one-source BConv formed inside the single-pass NTT serves more
    destination limbs and is pinned by the L = 24 Rescale tests and
    test_rescale_either_side_of_the_one_source_limit."""
    main, aux, L = Q30[:4], Q31[:1], 4
    param = chd.Param(main, aux, [(i, 0) for i in range(1, L + 1)])
    ctx = chd.Context(param)
    r = rng(470 + int(rescale))
    b1, a1, b2, a2 = (uniform_limbs(r, main) for _ in range(4))
    kb, ka = _evk(r, main, aux, L)
    out_l = L - 1 if rescale else L
    res = (zeros(out_l, N), zeros(out_l, N))
    ctx.hmult(L - 1, res, (dev(b1), dev(a1)), (dev(b2), dev(a2)),
              [dev(k) for k in kb], [dev(k) for k in ka], rescale=rescale)
    wb, wa = _orc.hmult(b1, a1, b2, a2, kb, ka, L, L, main, aux, 16,
                        1 if rescale else 0)
    assert np.array_equal(host(res[0]), wb)
    assert np.array_equal(host(res[1]), wa)
    if not rescale:
        out = (zeros(L - 1, N), zeros(L - 1, N))
        ctx.rescale(L - 1, out, res)
        assert np.array_equal(host(out[0]), _orc.rescale(wb, main, L, 1, 16))
        assert np.array_equal(host(out[1]), _orc.rescale(wa, main, L, 1, 16))


@pytest.mark.parametrize("L", [7, 8, 13, 14])
def test_rescale_either_side_of_the_one_source_limit(chd, ks, L):
    """Rescale has one source limb: up to 12 destination polynomial-limbs
    the BConv writes the destination and a two-pass NTT runs in place on
    it, above that the single-pass NTT forms the BConv as it reads. The
    ciphertext (2 x 6 = 12 limbs at L = 7, 2 x 7 = 14 at L = 8) and the
    single polynomial (12 at L = 13, 13 at L = 14) on both sides, against
    the oracle"""
    param, ctx, main, aux = ks
    r = rng(490 + L)
    b, a = uniform_limbs(r, main[:L]), uniform_limbs(r, main[:L])
    out = (zeros(L - 1, N), zeros(L - 1, N))
    ctx.rescale(L - 1, out, (dev(b), dev(a)))
    assert np.array_equal(host(out[0]), _orc.rescale(b, main, L, 1, 16))
    assert np.array_equal(host(out[1]), _orc.rescale(a, main, L, 1, 16))
    one = zeros(L - 1, N)
    ctx.rescale_poly(L - 1, one, dev(b))
    assert np.array_equal(host(one), _orc.rescale(b, main, L, 1, 16))


@pytest.mark.parametrize("L", [4, 24])
def test_rescale_rejects_result_overlapping_kept_limbs(chd, ks, L):
    """a Rescale whose result bx is the input's ax overlaps the kept source
    limbs the ModDown epilogue reads: the call fails before any launch
    (also where few destination limbs let the BConv write the destination
    first) and the input is left as it was"""
    param, ctx, main, aux = ks
    r = rng(480 + L)
    b, a = uniform_limbs(r, main[:L]), uniform_limbs(r, main[:L])
    tb, ta = dev(b), dev(a)
    out_a = zeros(L - 1, N)
    with pytest.raises(chd.ChdError, match="overlap"):
        ctx.rescale(L - 1, (ta[:L - 1], out_a), (tb, ta))
    assert np.array_equal(host(ta), a) and np.array_equal(host(tb), b)


def test_rescale_polynomials_in_any_order(chd, ks):
    """Rescale runs bx and ax together, addressing ax as bx plus their
    distance: here ax lies below bx in one buffer and the result's bx sits
    between them; both polynomials must match the oracle"""
    import torch
    param, ctx, main, aux = ks
    L = 24
    r = rng(460)
    b, a = uniform_limbs(r, main), uniform_limbs(r, main)
    big = zeros(4 * L, N)
    a_ax, res_bx = big[0:L], big[L:2 * L - 1]
    a_bx, res_ax = big[2 * L:3 * L], big[3 * L:4 * L - 1]
    a_ax.copy_(dev(a))
    a_bx.copy_(dev(b))
    ctx.rescale(L - 1, (res_bx, res_ax), (a_bx, a_ax))
    torch.cuda.synchronize()
    assert np.array_equal(host(res_bx), _orc.rescale(b, main, L, 1, 16))
    assert np.array_equal(host(res_ax), _orc.rescale(a, main, L, 1, 16))
    # the sources are untouched
    assert np.array_equal(host(a_bx), b) and np.array_equal(host(a_ax), a)


@pytest.mark.parametrize("rot", [1, 1234])
def test_hrot_and_mult_key(chd, ks, rot, L=20):
    param, ctx, main, aux = ks
    r = rng(500 + rot + 100 * L)
    b, a = uniform_limbs(r, main[:L]), uniform_limbs(r, main[:L])
    kb, ka = _evk(r, main, aux, 3)
    res = (zeros(L, N), zeros(L, N))
    ctx.mult_key(L - 1, res, (dev(b), dev(a)), [dev(k) for k in kb],
                 [dev(k) for k in ka])
    wb, wa = _orc.mult_key(b, a, kb, ka, L, 24, main, aux, 16)
    assert np.array_equal(host(res[0]), wb)
    assert np.array_equal(host(res[1]), wa)
    ctx.hrot(L - 1, res, (dev(b), dev(a)), [dev(k) for k in kb],
             [dev(k) for k in ka], rot)
    # HRot reduces the distance modulo the slot count (Context.cpp:776-791);
    # the oracle takes the permute amount itself
    hb, ha = _orc.hrot(b, a, kb, ka, L, 24, main, aux, 16, rot % (N // 2))
    assert np.array_equal(host(res[0]), hb)
    assert np.array_equal(host(res[1]), ha)


@pytest.mark.parametrize("L,rot", [(1, 3), (8, -1), (9, 77), (17, 4096)])
def test_hrot_mult_key_level_sweep(chd, ks, L, rot):
    """MultKey and HRot at the low levels (one group, partial last groups;
    negative and large rotations) against the oracle"""
    test_hrot_and_mult_key(chd, ks, rot, L)


def test_permute_conjugate(chd, ks):
    param, ctx, main, _ = ks
    L = 5
    r = rng(600)
    b, a = uniform_limbs(r, main[:L]), uniform_limbs(r, main[:L])
    res = (zeros(L, N), zeros(L, N))
    ctx.permute(L - 1, res, (dev(b), dev(a)), -1)
    g = 2 * N - 1
    assert np.array_equal(host(res[0]), _orc.permute(b, 16, g))
    assert np.array_equal(host(res[1]), _orc.permute(a, 16, g))


def test_hmult_alternating_streams(chd, ks):
    """Key switches issued back to back on two streams share the context's
    scratch arena; the second stream must wait for the first one's use."""
    import ctypes
    import torch
    param, ctx, main, aux = ks
    L = 24
    r = rng(470)
    kb, ka = _evk(r, main, aux, 3)
    dkb, dka = [dev(k) for k in kb], [dev(k) for k in ka]
    cases = []
    for _ in range(2):
        b1, a1, b2, a2 = (uniform_limbs(r, main) for _ in range(4))
        cases.append(((b1, a1, b2, a2), (dev(b1), dev(a1)), (dev(b2), dev(a2)),
                      (zeros(L - 1, N), zeros(L - 1, N))))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for rep in range(3):
        for i, (_, a, b, res) in enumerate(cases):
            s = ctypes.c_void_p(streams[i].cuda_stream)
            ctx.hmult(L - 1, res, a, b, dkb, dka, rescale=True, stream=s)
    torch.cuda.synchronize()
    for (b1, a1, b2, a2), _, _, res in cases:
        wb, wa = _orc.hmult(b1, a1, b2, a2, kb, ka, L, 24, main, aux, 16, 1)
        assert np.array_equal(host(res[0]), wb)
        assert np.array_equal(host(res[1]), wa)


# ------------------------------------------------------- hoisted rotations ----
def _rot_keys(r, main, aux, rots, beta=3):
    return {rot: _evk(r, main, aux, beta) for rot in rots}


def test_hoist_baby_steps_config5_level(chd, ks):
    """config-5 level (L = 20 of a 24-prime chain; keys skip 4 q limbs via
    the extra gap): every baby step bit-exact against the restatement"""
    import hoist_ref
    param, ctx, main, aux = ks
    L = 20
    r = rng(500)
    b, a = uniform_limbs(r, main[:L]), uniform_limbs(r, main[:L])
    rots = [0, 1, 2, 5, 27, 28, 29, 30, 31, 32]  # 9 non-zero: two launches
    keys = _rot_keys(r, main, aux, [x for x in rots if x])
    dkeys = {k: ([dev(x) for x in v[0]], [dev(x) for x in v[1]])
             for k, v in keys.items()}
    dst = [(zeros(L + 8, N), zeros(L + 8, N)) for _ in rots]
    ctx.hoist_baby_steps(L - 1, (dev(b), dev(a)), rots, dst, dkeys)
    modup = _orc.mod_up(a, main[:L], aux, 16)
    for rot, (db, da) in zip(rots, dst):
        wb, wa = hoist_ref.baby_step(b, a, keys.get(rot), rot, L, 24, main,
                                     aux, 16, modup)
        assert np.array_equal(host(db), wb), "rot %d b" % rot
        assert np.array_equal(host(da), wa), "rot %d a" % rot


def test_hoist_evaluate_config5_level(chd, ks):
    """double-hoisted BSGS at L = 20: 10 baby steps (two fused baby-step
    launches of up to 8 rotations, one accumulation chunk) and 3 giant
    steps; the one-shot entry point and a handler run twice (buffer reuse)
    on different ciphertexts"""
    import hoist_ref
    param, ctx, main, aux = ks
    L = 20
    r = rng(510)
    bsi, gsi = list(range(10)), [0, 10, 20]
    pts = {(g, s): uniform_limbs(r, main[:L] + aux) for g in gsi for s in bsi
           if (g, s) != (20, 9)}  # one absent plaintext
    keys = _rot_keys(r, main, aux, sorted(set(bsi[1:] + gsi[1:])))
    dkeys = {k: ([dev(x) for x in v[0]], [dev(x) for x in v[1]])
             for k, v in keys.items()}
    dpts = {k: dev(v) for k, v in pts.items()}
    cts = [(uniform_limbs(r, main[:L]), uniform_limbs(r, main[:L]))
           for _ in range(2)]
    wants = [hoist_ref.evaluate(b, a, pts, keys, L, 24, main, aux, 16)
             for b, a in cts]
    res = (zeros(L - 1, N), zeros(L - 1, N))
    ctx.hoist_evaluate(L - 1, res, (dev(cts[0][0]), dev(cts[0][1])), gsi, bsi,
                       dpts, dkeys)
    assert np.array_equal(host(res[0]), wants[0][0])
    assert np.array_equal(host(res[1]), wants[0][1])
    h = chd.Hoist(ctx, L - 1, gsi, bsi, dpts)
    for (b, a), (wb, wa) in zip(cts, wants):
        out = (zeros(L - 1, N), zeros(L - 1, N))
        h.run(out, (dev(b), dev(a)), dkeys)
        assert np.array_equal(host(out[0]), wb)
        assert np.array_equal(host(out[1]), wa)


@pytest.mark.parametrize("L", [20, 21])
def test_hoist_evaluate_many_giant_steps(chd, ks, L):
    """12 giant steps at L = 20 and 21: the wide giant-step accumulation
    (every giant step in each launch, padded to 16 rows that are skipped;
    launches of two limbs, the last of one limb at L = 21's 29 limbs) and
    the batched giant-step key switches (a batch of 8 and one of 3), with
    absent pairs"""
    import hoist_ref
    param, ctx, main, aux = ks
    r = rng(520 + L)
    bsi, gsi = [0, 1, 2], [3 * k for k in range(12)]
    pts = {(g, s): uniform_limbs(r, main[:L] + aux) for g in gsi for s in bsi
           if (g, s) not in ((6, 1), (33, 2))}
    keys = _rot_keys(r, main, aux, sorted(set(bsi[1:] + gsi[1:])))
    dkeys = {k: ([dev(x) for x in v[0]], [dev(x) for x in v[1]])
             for k, v in keys.items()}
    dpts = {k: dev(v) for k, v in pts.items()}
    b, a = uniform_limbs(r, main[:L]), uniform_limbs(r, main[:L])
    wb, wa = hoist_ref.evaluate(b, a, pts, keys, L, 24, main, aux, 16)
    h = chd.Hoist(ctx, L - 1, gsi, bsi, dpts)
    out = (zeros(L - 1, N), zeros(L - 1, N))
    h.run(out, (dev(b), dev(a)), dkeys)
    assert np.array_equal(host(out[0]), wb)
    assert np.array_equal(host(out[1]), wa)
    # the handle keeps these plaintexts only in its tiled array: the min_ks
    # order takes each giant step's row back out of it
    mb, ma = hoist_ref.evaluate_min_ks(b, a, pts, keys, L, 24, main, aux, 16)
    assert h.required_rotations(min_ks=True) == [1, 3]
    out = (zeros(L - 1, N), zeros(L - 1, N))
    h.run(out, (dev(b), dev(a)), dkeys, min_ks=True)
    assert np.array_equal(host(out[0]), mb)
    assert np.array_equal(host(out[1]), ma)


def test_gs_tiled_pack_and_untile(chd):
    """chd_k_gs_pack_tiled puts word c of block k of limb l of plaintext
    (g, b) at ((((l * 256 + k) * rows + g) * stride + b) << 8) + c (checked
    word by word on the host), and chd_k_gs_untile_row gives each row's
    plaintexts back, whole or their first limbs"""
    import torch
    lib = chd.lib
    P = ctypes.c_void_p
    lib.chd_k_gs_pack_tiled.argtypes = [P, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, P, P]
    lib.chd_k_gs_untile_row.argtypes = [P, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, P, P]
    rows, stride, limbs = 3, 4, 5
    r = rng(540)
    pts = [[r.integers(0, 1 << 32, (limbs, N), dtype=np.uint64).astype(
        np.uint32) for _ in range(stride)] for _ in range(rows)]
    dpts = [[dev(x) for x in row] for row in pts]
    table = torch.tensor([t.data_ptr() for row in dpts for t in row],
                         dtype=torch.int64, device="cuda")
    tiled = torch.empty(rows * stride * limbs * N, dtype=torch.int32,
                        device="cuda")
    assert lib.chd_k_gs_pack_tiled(P(table.data_ptr()), rows, stride, limbs,
                                   P(tiled.data_ptr()), None) == 0
    got = host(tiled).reshape(limbs, N >> 8, rows, stride, 256)
    want = np.stack([np.stack(row) for row in pts])  # g, b, l, n
    want = want.reshape(rows, stride, limbs, N >> 8, 256).transpose(2, 3, 0,
                                                                  1, 4)
    assert np.array_equal(got, want)
    for g in range(rows):
        for dl in (limbs, 2):
            out = zeros(stride * dl, N)
            assert lib.chd_k_gs_untile_row(P(tiled.data_ptr()), rows, stride,
                                           limbs, g, dl, P(out.data_ptr()),
                                           None) == 0
            back = host(out).reshape(stride, dl, N)
            for b in range(stride):
                assert np.array_equal(back[b], pts[g][b][:dl]), (g, dl, b)


def test_hoist_evaluate_chunked_accumulation(chd, ks):
    """36 baby steps x 9 giant steps at L = 20: more baby steps than one
    accumulation launch takes (32), so the second chunk adds onto the first
    one's sums (add_to_dst), and more giant steps than one launch holds (8),
    so two giant-step launches and two batches of giant-step key switches
    run; with absent pairs"""
    import hoist_ref
    param, ctx, main, aux = ks
    L = 20
    r = rng(530)
    bsi, gsi = list(range(36)), [36 * k for k in range(9)]
    pts = {(g, s): uniform_limbs(r, main[:L] + aux) for g in gsi for s in bsi
           if (g, s) not in ((36, 33), (288, 2), (144, 0))}
    keys = _rot_keys(r, main, aux, sorted(set(bsi[1:] + gsi[1:])))
    dkeys = {k: ([dev(x) for x in v[0]], [dev(x) for x in v[1]])
             for k, v in keys.items()}
    dpts = {k: dev(v) for k, v in pts.items()}
    b, a = uniform_limbs(r, main[:L]), uniform_limbs(r, main[:L])
    print("hoist 36 baby x 9 giant steps", flush=True)
    h = chd.Hoist(ctx, L - 1, gsi, bsi, dpts)
    out = (zeros(L - 1, N), zeros(L - 1, N))
    h.run(out, (dev(b), dev(a)), dkeys)
    got_b, got_a = host(out[0]), host(out[1])
    del dpts, dkeys
    _orc.lib.orc_set_threads(8)
    wb, wa = hoist_ref.evaluate(b, a, pts, keys, L, 24, main, aux, 16)
    assert np.array_equal(got_b, wb)
    assert np.array_equal(got_a, wa)
