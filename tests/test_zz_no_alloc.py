"""chd_hmult_noalloc, the HMult entry point that allocates nothing (no
counterpart in the reference; for callers that cannot allocate device
memory), against chd_hmult through the C-ABI: bit-exact on consecutive
calls, the second on a smaller input (the static scratch array keeps the
previous call's contents), with and without the merged rescale, and no
change of the device's free memory across the calls. A level whose
temporaries exceed the static array is rejected with an error."""
import numpy as np
import pytest

from gpu_util import N, Q30, Q31, config4, dev, host, uniform_limbs, zeros

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def chd():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("no HIP device visible")
    import cheddar_amd
    return cheddar_amd


def _inputs(r, main, aux, L, beta=3):
    q = main[:L]
    a = (dev(uniform_limbs(r, q)), dev(uniform_limbs(r, q)))
    b = (dev(uniform_limbs(r, q)), dev(uniform_limbs(r, q)))
    kb = [dev(uniform_limbs(r, main + aux)) for _ in range(beta)]
    ka = [dev(uniform_limbs(r, main + aux)) for _ in range(beta)]
    return a, b, kb, ka


def test_hmult_noalloc_matches_hmult(chd):
    import torch
    main, aux, levels = config4()
    ctx = chd.Context(chd.Param(main, aux, levels))
    r = np.random.default_rng(0xA110C)
    free = []
    # top level first, then a smaller input; the last call without rescale
    for level, rescale in ((23, True), (19, True), (19, False)):
        print("hmult_noalloc level", level, "rescale", rescale, flush=True)
        a, b, kb, ka = _inputs(r, main, aux, level + 1)
        out_l = level + 1 - int(rescale)
        want = (zeros(out_l, N), zeros(out_l, N))
        got = (zeros(out_l, N), zeros(out_l, N))
        ctx.hmult(level, want, a, b, kb, ka, rescale=rescale)
        torch.cuda.synchronize()
        free.append(torch.cuda.mem_get_info()[0])
        ctx.hmult_noalloc(level, got, a, b, kb, ka, rescale=rescale)
        torch.cuda.synchronize()
        free.append(torch.cuda.mem_get_info()[0])
        assert np.array_equal(host(got[0]), host(want[0]))
        assert np.array_equal(host(got[1]), host(want[1]))
    # the first call may load the library's code object that holds the
    # static array; from then on no call changes the free device memory
    assert free[2] == free[3] and free[4] == free[5]


def test_hmult_noalloc_result_may_alias_input(chd):
    main, aux, levels = config4()
    ctx = chd.Context(chd.Param(main, aux, levels))
    r = np.random.default_rng(0xA110D)
    level = 21
    a, b, kb, ka = _inputs(r, main, aux, level + 1)
    want = (zeros(level, N), zeros(level, N))
    ctx.hmult(level, want, a, b, kb, ka)
    ctx.hmult_noalloc(level, a, a, b, kb, ka)  # res = a, as HMult allows
    assert np.array_equal(host(a[0])[:level], host(want[0]))
    assert np.array_equal(host(a[1])[:level], host(want[1]))


def test_hmult_noalloc_two_contexts_two_streams(chd):
    """two contexts share the GPU's one static array; their calls, issued
    back to back on two streams without any ordering by the caller, are
    ordered by the library and stay bit-exact against chd_hmult"""
    import ctypes
    import torch
    main, aux, levels = config4()
    ctxs = [chd.Context(chd.Param(main, aux, levels)) for _ in range(2)]
    r = np.random.default_rng(0xA110F)
    jobs = []
    for ctx, level in zip(ctxs, (23, 20)):
        a, b, kb, ka = _inputs(r, main, aux, level + 1)
        want = (zeros(level, N), zeros(level, N))
        ctx.hmult(level, want, a, b, kb, ka)
        jobs.append((ctx, level, a, b, kb, ka, want,
                     [(zeros(level, N), zeros(level, N)) for _ in range(3)]))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in range(2)]
    for rep in range(3):
        for (ctx, level, a, b, kb, ka, _, got), st in zip(jobs, streams):
            print("hmult_noalloc two contexts: level", level, "call", rep,
                  flush=True)
            ctx.hmult_noalloc(level, got[rep], a, b, kb, ka,
                              stream=ctypes.c_void_p(st.cuda_stream))
    torch.cuda.synchronize()
    for ctx, level, a, b, kb, ka, want, got in jobs:
        for g in got:
            assert np.array_equal(host(g[0]), host(want[0])), level
            assert np.array_equal(host(g[1]), host(want[1])), level


def test_hmult_noalloc_rejects_levels_beyond_its_scratch(chd):
    """30 q limbs with alpha = 8 need about 69 MiB of temporaries"""
    main, aux = Q30[:30], Q31[:8]
    ctx = chd.Context(chd.Param(main, aux, [(i, 0) for i in range(1, 31)]))
    r = np.random.default_rng(0xA110E)
    a, b, kb, ka = _inputs(r, main, aux, 30, beta=4)
    res = (zeros(29, N), zeros(29, N))
    with pytest.raises(chd.ChdError, match="MiB of scratch"):
        ctx.hmult_noalloc(29, res, a, b, kb, ka)
    ctx.hmult_noalloc(24, (zeros(24, N), zeros(24, N)), a, b, kb, ka)
