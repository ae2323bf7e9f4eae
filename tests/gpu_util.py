"""Helpers for GPU parity tests: numpy <-> torch device transfers and the
configuration prime chains. Test infrastructure only."""
import numpy as np

from chd_primes import ntt_primes

N = 1 << 16
CFG1_Q = 2147352577
Q30 = ntt_primes(30, 32)        # config-2 chain / config-4 main primes
Q31 = ntt_primes(31, 48)        # config-3 targets / config-4 special primes


def dev(a):
    import torch
    a = np.ascontiguousarray(a, dtype=np.uint32)
    return torch.from_numpy(a.view(np.int32)).to("cuda")


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.detach().cpu().numpy().view(np.uint32)


def zeros(*shape):
    import torch
    return torch.zeros(*shape, dtype=torch.int32, device="cuda")


def uniform_limbs(rng, primes, n=N):
    return np.stack([rng.integers(0, p, n, dtype=np.uint64).astype(np.uint32)
                     for p in primes])


def centred_limbs(rng, primes, n=N):
    return np.stack([rng.integers(-((p - 1) // 2), (p - 1) // 2 + 1, n)
                     .astype(np.int32) for p in primes])


def config4(L=24):
    """main = 30-bit primes [0..L), aux = 31-bit [0..8), one level per
    prime count (level_config [[1,0],...,[L,0]])"""
    main = Q30[:L]
    aux = Q31[:8]
    levels = [(i, 0) for i in range(1, L + 1)]
    return main, aux, levels
