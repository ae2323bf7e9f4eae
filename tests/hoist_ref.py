"""CPU restatement of the hoisted baby-step / giant-step evaluation
(src/extension/Hoist.cu:578-691 baby step with BSFusedKeyMult,
840-975 EvaluateGiantStepOptimized, 487-515 EvaluateFinalModDown), composed
from the oracle's primitives (ModUp, PAccum, ModDown, Permute, MontMul).

Test infrastructure only: the checker for the hoisting kernels.
Limb arrays are NTT-domain Montgomery residues [limbs][N].
"""
import numpy as np

import _orc
from ckks_host import mont_mul_vec


def _mul(a, b, primes):
    out = np.empty_like(a)
    for i, p in enumerate(primes):
        out[i] = mont_mul_vec(a[i], b[i], p)
    return out


def _add(a, b, primes):
    out = np.empty_like(a)
    for i, p in enumerate(primes):
        out[i] = ((a[i].astype(np.uint64) + b[i]) % p).astype(np.uint32)
    return out


def pseudo_mod_up(x, q_primes, p_primes):
    """ModSwitch.cu:414-428: MontMul(x, ToMont(P mod q)) on the q limbs,
    zero-extended over the alpha aux limbs (Hoist.cu:631-646)."""
    pp = _orc.p_prod(q_primes, p_primes)
    n = x.shape[1]
    out = np.zeros((len(q_primes) + len(p_primes), n), np.uint32)
    for i, q in enumerate(q_primes):
        out[i] = mont_mul_vec(x[i], np.full(n, pp[i], np.uint32), q)
    return out


def paccum(modup, key_b, key_a, L, max_q, q_primes, p_primes, log_n):
    """sum over dnum groups of MontMul(modup_g, key_g) on L + alpha limbs
    (MultKeyNoModDown without CAccum, Context.cpp:609-643)"""
    alpha = len(p_primes)
    beta = modup.shape[0]
    n = 1 << log_n
    primes = list(q_primes[:L]) + list(p_primes)
    acc_b = np.zeros((L + alpha, n), np.uint32)
    acc_a = np.zeros((L + alpha, n), np.uint32)
    _orc.lib.orc_paccum(acc_b, acc_a, _orc.u32(modup), beta, _orc.u32(key_b),
                        _orc.u32(key_a), L, alpha, max_q, _orc.u32(primes),
                        log_n)
    return acc_b, acc_a


def baby_step(ct_b, ct_a, key, rot, L, max_q, q_primes, p_primes, log_n,
              modup=None):
    """extended-basis baby step for rotation rot (Hoist.cu:20-78, 578-691);
    modup: the ModUp of ct_a when already computed (it is hoisted)"""
    q = list(q_primes[:L])
    p = list(p_primes)
    primes = q + p
    if rot == 0:
        return pseudo_mod_up(ct_b, q, p), pseudo_mod_up(ct_a, q, p)
    if modup is None:
        modup = _orc.mod_up(ct_a, q, p, log_n)
    tb, ta = paccum(modup, key[0], key[1], L, max_q, q, p, log_n)
    tb = _add(tb, pseudo_mod_up(ct_b, q, p), primes)
    g = _orc.lib.orc_galois_factor(rot, log_n)
    return _orc.permute(tb, log_n, g), _orc.permute(ta, log_n, g)


def evaluate(ct_b, ct_a, pts, keys, L, max_q, q_primes, p_primes, log_n):
    """res = ModDownAndRescale(sum_g Rot_g(sum_b pt[g, b] * bs[b])) with the
    giant steps' double hoisting. pts: {(g, b): L + alpha limbs}; keys:
    {rot: (key_b, key_a)} (any mappings: each plaintext is read once, each
    key's pair used before the next key is looked up). Returns (res_b,
    res_a) of L - 1 limbs."""
    q = list(q_primes[:L])
    p = list(p_primes)
    primes = q + p
    n = 1 << log_n
    bs_idx = sorted({b for (_, b) in pts})
    gs_idx = sorted({g for (g, _) in pts})
    modup = _orc.mod_up(ct_a, q, p, log_n)
    bs = {b: baby_step(ct_b, ct_a, keys.get(b), b, L, max_q, q, p, log_n,
                       modup) for b in bs_idx}
    acc = {}
    for g in gs_idx:
        ab = np.zeros((L + len(p), n), np.uint32)
        aa = np.zeros_like(ab)
        for b in bs_idx:
            if (g, b) not in pts:
                continue
            pt = pts[(g, b)]
            _orc.pmult_accum(ab, pt, bs[b][0], primes, log_n)
            _orc.pmult_accum(aa, pt, bs[b][1], primes, log_n)
        acc[g] = (ab, aa)
    fb = acc[0][0] if 0 in acc else np.zeros((L + len(p), n), np.uint32)
    fa = acc[0][1] if 0 in acc else np.zeros((L + len(p), n), np.uint32)
    for g in gs_idx:
        if g == 0:
            continue
        d = _orc.mod_down(acc[g][1], primes, L, log_n)
        modup = _orc.mod_up(d, q, p, log_n)
        tb, ta = paccum(modup, keys[g][0], keys[g][1], L, max_q, q, p, log_n)
        tb = _add(tb, acc[g][0], primes)
        gal = _orc.lib.orc_galois_factor(g, log_n)
        fb = _add(fb, _orc.permute(tb, log_n, gal), primes)
        fa = _add(fa, _orc.permute(ta, log_n, gal), primes)
    rb = _orc.mod_down(fb, primes, L - 1, log_n)
    ra = _orc.mod_down(fa, primes, L - 1, log_n)
    return rb, ra


def evaluate_gs_only(ct_b, ct_a, pts, keys, L, max_q, q_primes, p_primes,
                     log_n):
    """maps whose giant steps hold only baby step 0 (Hoist.cu:715-797), in
    the reference's order: for g != 0 the key switch of ct with key g plus
    P * ct_b, multiplied by pt_g, then permuted by g; for g == 0 the P-raised
    ct times pt_0; the sum brought down by ModDownAndRescale.
    pts: {g: L + alpha limbs}."""
    q = list(q_primes[:L])
    p = list(p_primes)
    primes = q + p
    n = 1 << log_n
    modup = _orc.mod_up(ct_a, q, p, log_n)
    pb = pseudo_mod_up(ct_b, q, p)
    fb = np.zeros((L + len(p), n), np.uint32)
    fa = np.zeros_like(fb)
    for g, pt in sorted(pts.items()):
        if g == 0:
            tb, ta = pb, pseudo_mod_up(ct_a, q, p)
        else:
            tb, ta = paccum(modup, keys[g][0], keys[g][1], L, max_q, q, p,
                            log_n)
            tb = _add(tb, pb, primes)
        tb, ta = _mul(tb, pt, primes), _mul(ta, pt, primes)
        if g != 0:
            gal = _orc.lib.orc_galois_factor(g, log_n)
            tb, ta = _orc.permute(tb, log_n, gal), _orc.permute(ta, log_n, gal)
        fb, fa = _add(fb, tb, primes), _add(fa, ta, primes)
    rb = _orc.mod_down(fb, primes, L - 1, log_n)
    ra = _orc.mod_down(fa, primes, L - 1, log_n)
    return rb, ra


def evaluate_min_ks(ct_b, ct_a, pts, keys, L, max_q, q_primes, p_primes,
                    log_n):
    """min_ks (Hoist.cu:517-566): bs[0] = ct, bs[k s] = HRot(bs[(k-1) s], s);
    giant steps from the last down: acc = sum_b pt[g, b] * bs[b] (q limbs of
    each plaintext) plus the running sum, HRot by the giant-step stride
    unless g == 0; then Rescale. keys: {stride: (key_b, key_a)}."""
    import math
    q = list(q_primes[:L])
    bs_idx = sorted({b for (_, b) in pts})
    gs_idx = sorted({g for (g, _) in pts})
    bs_stride = math.gcd(*[b for b in bs_idx if b] or [0])
    gs_stride = math.gcd(*[g for g in gs_idx if g] or [0])
    bs = {0: (ct_b, ct_a)}
    for b in bs_idx:
        if b == 0:
            continue
        pb, pa = bs[b - bs_stride]
        bs[b] = _orc.hrot(pb, pa, keys[bs_stride][0], keys[bs_stride][1], L,
                          max_q, q_primes, p_primes, log_n, bs_stride)
    acc = None
    for g in reversed(gs_idx):
        ab = np.zeros_like(ct_b) if acc is None else acc[0]
        aa = np.zeros_like(ct_a) if acc is None else acc[1]
        for b in bs_idx:
            if (g, b) not in pts:
                continue
            pt = pts[(g, b)][:L]
            ab = _add(ab, _mul(pt, bs[b][0], q), q)
            aa = _add(aa, _mul(pt, bs[b][1], q), q)
        if g != 0:
            ab, aa = _orc.hrot(ab, aa, keys[gs_stride][0], keys[gs_stride][1],
                               L, max_q, q_primes, p_primes, log_n, gs_stride)
        acc = (ab, aa)
    rb = _orc.rescale(acc[0], q_primes, L, 1, log_n)
    ra = _orc.rescale(acc[1], q_primes, L, 1, log_n)
    return rb, ra
