"""ctypes binding of the CPU oracle (oracle/_build/liboracle.so) for the tests.

Test infrastructure: the oracle is the checker, never the thing measured.
"""
import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
LIB_PATH = os.path.join(ORACLE_DIR, "_build", "liboracle.so")

_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u32 = ctypes.c_uint32
_i32 = ctypes.c_int32
_int = ctypes.c_int


def _load():
    if not os.path.exists(LIB_PATH):
        subprocess.check_call(["make", "-s", "-C", ORACLE_DIR])
    lib = ctypes.CDLL(LIB_PATH)
    sig = {
        "orc_mulmod": (_u32, [_u32, _u32, _u32]),
        "orc_powmod": (_u32, [_u32, ctypes.c_int64, _u32]),
        "orc_invmod": (_u32, [_u32, _u32]),
        "orc_find_generator": (_u32, [_u32]),
        "orc_primitive_root": (_u32, [_u32, _u32]),
        "orc_inv_mod_base": (_i32, [_u32]),
        "orc_to_mont": (_u32, [_u32, _u32]),
        "orc_mont_mul": (_u32, [_u32, _u32, _u32]),
        "orc_bitrev": (_u32, [_u32, _int]),
        "orc_twiddles": (None, [_u32, _int, _u32p, _u32p, _u32p]),
        "orc_ntt": (None, [_u32p, _int, _u32, _int]),
        "orc_ntt_exact": (None, [_u32p, _int, _u32, _int]),
        "orc_intt": (None, [_u32p, _int, _u32, _int]),
        "orc_intt_exact": (None, [_u32p, _int, _u32, _int]),
        "orc_intt_mult_const": (None, [_i32p, _u32p, _int, _u32, _u32, _int]),
        "orc_set_threads": (None, [_int]),
        "orc_ntt_batch": (None, [_u32p, _int, _int, _u32p, _int]),
        "orc_intt_batch": (None, [_u32p, _int, _int, _u32p, _int]),
        "orc_bconv": (None, [_u32p, _i32p, _int, _int, _i32p, _u32p, _int]),
        "orc_modswitch_consts": (None, [_u32p, _int, _u32p, _int, _int, _int,
                                        _int, _u32p, _i32p]),
        "orc_moddown_epilogue_consts": (None, [_u32p, _int, _u32p, _int, _int,
                                               _int, _u32p, _u32p]),
        "orc_mod_up": (_int, [_u32p, _u32p, _int, _u32p, _u32p, _int, _int]),
        "orc_mod_down": (None, [_u32p, _u32p, _int, _u32p, _int, _int]),
        "orc_mod_up_ex": (_int, [_u32p, _u32p, _int, _u32p, _u32p, _int, _int,
                                 _int]),
        "orc_mod_down_ex": (None, [_u32p, _u32p, _u32p, _i32p, _int, _u32p,
                                   _int, _i32p, _int]),
        "orc_paccum_ex": (None, [_u32p, _u32p, _u32p, _int, _i32p, _u32p,
                                 _u32p, _int, _int, _int, _int, _u32p, _int]),
        "orc_tensor": (None, [_u32p] * 7 + [_int, _u32p, _int]),
        "orc_paccum": (None, [_u32p, _u32p, _u32p, _int, _u32p, _u32p, _int,
                              _int, _int, _u32p, _int]),
        "orc_caccum": (None, [_u32p, _u32p, _u32p, _int, _u32p, _int]),
        "orc_pmult_accum": (None, [_u32p, _u32p, _u32p, _int, _u32p, _int]),
        "orc_p_prod": (None, [_u32p, _u32p, _int, _u32p, _int]),
        "orc_permute": (None, [_u32p, _u32p, _int, _int, _u32]),
        "orc_galois_factor": (_u32, [_int, _int]),
        "orc_hmult": (_int, [_u32p] * 8 + [_int, _int, _u32p, _u32p, _int,
                                           _int, _int]),
        "orc_rescale": (_int, [_u32p, _u32p, _int, _u32p, _int, _int]),
        "orc_mult_key": (_int, [_u32p] * 6 + [_int, _int, _u32p, _u32p, _int,
                                              _int]),
        "orc_hrot": (_int, [_u32p] * 6 + [_int, _int, _u32p, _u32p, _int, _int,
                                          _int]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


lib = _load()


def u32(a):
    return np.ascontiguousarray(a, dtype=np.uint32)


def twiddles(q, log_n):
    n = 1 << log_n
    pr = np.zeros(n, np.uint32)
    pir = np.zeros(n, np.uint32)
    c = np.zeros(5, np.uint32)
    lib.orc_twiddles(q, log_n, pr, pir, c)
    return pr, pir, c


def ntt(x, log_n, q, mont=0, exact=False):
    y = u32(x).copy()
    (lib.orc_ntt_exact if exact else lib.orc_ntt)(y, log_n, q, mont)
    return y


def intt(x, log_n, q, mont=1, exact=False):
    y = u32(x).copy()
    (lib.orc_intt_exact if exact else lib.orc_intt)(y, log_n, q, mont)
    return y


def ntt_batch(x, log_n, primes, mont=0):
    y = u32(x).copy()
    lib.orc_ntt_batch(y, len(primes), log_n, u32(primes), mont)
    return y


def intt_batch(x, log_n, primes, mont=1):
    y = u32(x).copy()
    lib.orc_intt_batch(y, len(primes), log_n, u32(primes), mont)
    return y


def intt_mult_const(x, log_n, q, c, normalize):
    out = np.zeros(1 << log_n, np.int32)
    lib.orc_intt_mult_const(out, u32(x), log_n, q, c, normalize)
    return out


def modswitch_consts(src, dst, log_n):
    c1 = np.zeros(len(src), np.uint32)
    c2 = np.zeros(len(src) * len(dst), np.int32)
    lib.orc_modswitch_consts(u32(src), len(src), u32(dst), len(dst), log_n, 0,
                             0, c1, c2)
    return c1, c2.reshape(len(dst), len(src))


def moddown_consts(src, dst):
    inv = np.zeros(len(dst), np.uint32)
    pad = np.zeros(len(dst), np.uint32)
    lib.orc_moddown_epilogue_consts(u32(src), len(src), u32(dst), len(dst), 0,
                                    0, inv, pad)
    return inv, pad


def bconv(src_centred, table, dst_primes, log_n):
    src = np.ascontiguousarray(src_centred, dtype=np.int32)
    table = np.ascontiguousarray(table, dtype=np.int32)
    dst = np.zeros((len(dst_primes), 1 << log_n), np.uint32)
    lib.orc_bconv(dst, src, table.shape[1], len(dst_primes), table,
                  u32(dst_primes), log_n)
    return dst


def mod_up(src, q_primes, p_primes, log_n):
    L, alpha = len(q_primes), len(p_primes)
    beta = (L + alpha - 1) // alpha
    dst = np.zeros((beta, L + alpha, 1 << log_n), np.uint32)
    lib.orc_mod_up(dst, u32(src), L, u32(q_primes), u32(p_primes), alpha,
                   log_n)
    return dst


def mod_up_ex(src, q_primes, p_primes, prime_offset, log_n):
    """ModUp with the chain's group layout: (beta, L + alpha, N) array, the
    empty groups (ending at or before prime_offset) zero"""
    L, alpha = len(q_primes), len(p_primes)
    beta = (L + prime_offset + alpha - 1) // alpha
    dst = np.zeros((beta, L + alpha, 1 << log_n), np.uint32)
    lib.orc_mod_up_ex(dst, u32(src), L, u32(q_primes), u32(p_primes), alpha,
                      prime_offset, log_n)
    return dst


def mod_down_ex(src, src_primes, drop, dst_primes, dst_src, log_n):
    """general ModDown: drop = source limb indices divided out; dst_src[k] =
    source limb kept in destination limb k, or -1 for a restored prime"""
    dst = np.zeros((len(dst_primes), 1 << log_n), np.uint32)
    lib.orc_mod_down_ex(dst, u32(src), u32(src_primes),
                        np.ascontiguousarray(drop, np.int32), len(drop),
                        u32(dst_primes), len(dst_primes),
                        np.ascontiguousarray(dst_src, np.int32), log_n)
    return dst


def paccum_ex(modup, key_group, key_b, key_a, L, alpha, max_q, key_off,
              primes, log_n):
    n = 1 << log_n
    acc_b = np.zeros((L + alpha, n), np.uint32)
    acc_a = np.zeros((L + alpha, n), np.uint32)
    lib.orc_paccum_ex(acc_b, acc_a, u32(modup), len(key_group),
                      np.ascontiguousarray(key_group, np.int32), u32(key_b),
                      u32(key_a), L, alpha, max_q, key_off, u32(primes), log_n)
    return acc_b, acc_a


def mod_down(src, src_primes, dst_len, log_n):
    dst = np.zeros((dst_len, 1 << log_n), np.uint32)
    lib.orc_mod_down(dst, u32(src), len(src_primes), u32(src_primes), dst_len,
                     log_n)
    return dst


def tensor(b1, a1, b2, a2, primes, log_n):
    shape = (len(primes), 1 << log_n)
    bx, ax, rx = (np.zeros(shape, np.uint32) for _ in range(3))
    lib.orc_tensor(bx, ax, rx, u32(b1), u32(a1), u32(b2), u32(a2), len(primes),
                   u32(primes), log_n)
    return bx, ax, rx


def permute(src, log_n, galois):
    src = u32(src)
    dst = np.zeros_like(src)
    lib.orc_permute(dst, src, src.size >> log_n, log_n, galois)
    return dst


def pmult_accum(acc, pt, x, primes, log_n):
    """acc += MontMul(pt, x) limb by limb, in place (acc: uint32 C array)"""
    assert acc.dtype == np.uint32 and acc.flags["C_CONTIGUOUS"]
    lib.orc_pmult_accum(acc, u32(pt), u32(x), len(primes), u32(primes), log_n)
    return acc


def p_prod(q_primes, p_primes):
    out = np.zeros(len(q_primes), np.uint32)
    lib.orc_p_prod(out, u32(q_primes), len(q_primes), u32(p_primes),
                   len(p_primes))
    return out


def hmult(b1, a1, b2, a2, key_b, key_a, L, max_q, q_primes, p_primes, log_n,
          rescale):
    n = 1 << log_n
    out_l = L - rescale
    rb = np.zeros((out_l, n), np.uint32)
    ra = np.zeros((out_l, n), np.uint32)
    lib.orc_hmult(rb, ra, u32(b1), u32(a1), u32(b2), u32(a2), u32(key_b),
                  u32(key_a), L, max_q, u32(q_primes), u32(p_primes),
                  len(p_primes), log_n, rescale)
    return rb, ra


def rescale(src, q_primes, L, drop, log_n):
    out = np.zeros((L - drop, 1 << log_n), np.uint32)
    lib.orc_rescale(out, u32(src), L, u32(q_primes), drop, log_n)
    return out


def mult_key(b, a, key_b, key_a, L, max_q, q_primes, p_primes, log_n):
    n = 1 << log_n
    rb = np.zeros((L, n), np.uint32)
    ra = np.zeros((L, n), np.uint32)
    lib.orc_mult_key(rb, ra, u32(b), u32(a), u32(key_b), u32(key_a), L, max_q,
                     u32(q_primes), u32(p_primes), len(p_primes), log_n)
    return rb, ra


def hrot(b, a, key_b, key_a, L, max_q, q_primes, p_primes, log_n, rot):
    n = 1 << log_n
    rb = np.zeros((L, n), np.uint32)
    ra = np.zeros((L, n), np.uint32)
    lib.orc_hrot(rb, ra, u32(b), u32(a), u32(key_b), u32(key_a), L, max_q,
                 u32(q_primes), u32(p_primes), len(p_primes), log_n, rot)
    return rb, ra
