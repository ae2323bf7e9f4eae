"""Deterministic NTT-friendly prime chains for the benchmark configurations.

q = k * 2^17 + 1 prime, searched downward from a bit bound, so every prime
supports negacyclic NTTs of any degree up to 2^16. The reference keeps its
prime chains in JSON parameter files (parameters/bootparam_30.json); this
helper regenerates the same kind of chain deterministically for the
synthetic workloads.
"""

_MR_BASES = (2, 3, 5, 7, 11, 13, 17)  # deterministic for n < 3.4e14


def is_prime(n):
    if n < 2:
        return False
    for p in _MR_BASES:
        if n % p == 0:
            return n == p
    d, s = n - 1, 0
    while d % 2 == 0:
        d //= 2
        s += 1
    for a in _MR_BASES:
        x = pow(a, d, n)
        if x in (1, n - 1):
            continue
        for _ in range(s - 1):
            x = x * x % n
            if x == n - 1:
                break
        else:
            return False
    return True


def ntt_primes(bits, count, log_two_n=17, skip=0):
    """The `count` largest primes q < 2^bits with q = 1 mod 2^log_two_n,
    after skipping the first `skip` of them, in descending order."""
    step = 1 << log_two_n
    q = ((1 << bits) - 1) // step * step + 1
    out = []
    while len(out) < count + skip:
        if q < (1 << (bits - 1)):
            raise ValueError("ran out of %d-bit primes" % bits)
        if is_prime(q):
            out.append(q)
        q -= step
    return out[skip:]
