"""Key-switch compositions for any level of a parameter set, terminal primes
included, restated from the reference over the oracle's primitives
(Context.cpp:584-871 HMult / MultKey / HRot / Rescale, ModSwitch.cu:175-684
ModUp / ModDown / BitPacker restore). Test infrastructure only.

A level's q limbs are the chain positions [off, off + L) of
chain = terminal primes reversed + main primes, off = max_ter - num_ter.
Keys hold max_q = max_ter + max_main q limbs (chain order) and alpha aux
limbs per dnum group; a level reads key limbs from off (Container.h's
extra_ view, Context.cpp:640).
"""
import numpy as np

import _orc
from ckks_host import mont_mul_vec


class Chain:
    def __init__(self, main, ter, aux, level_config, log_n=16):
        self.main = [int(p) for p in main]
        self.ter = [int(p) for p in ter]
        self.aux = [int(p) for p in aux]
        self.levels = [tuple(c) for c in level_config]
        self.log_n = log_n
        self.max_ter, self.max_main = len(self.ter), len(self.main)
        self.alpha = len(self.aux)
        self.max_q = self.max_ter + self.max_main
        self.chain = self.ter[::-1] + self.main

    def np(self, level):
        return self.levels[level]            # (num_main, num_ter)

    def offset(self, level):
        return self.max_ter - self.np(level)[1]

    def q(self, level):
        m, t = self.np(level)
        return self.chain[self.max_ter - t: self.max_ter + m]

    def groups(self, level):
        """absolute dnum groups that hold limbs of this level"""
        L, off = len(self.q(level)), self.offset(level)
        beta = (L + off + self.alpha - 1) // self.alpha
        return [g for g in range(beta)
                if min((g + 1) * self.alpha, L + off) > off]

    # ------------------------------------------------------------ pieces
    def mod_up(self, x, level):
        """non-empty groups of the ModUp of x, stacked"""
        full = _orc.mod_up_ex(x, self.q(level), self.aux, self.offset(level),
                              self.log_n)
        return full[self.groups(level)]

    def key_mult(self, d, level, key_b, key_a):
        """PAccum of ModUp(d) with the key over L + alpha limbs"""
        q = self.q(level)
        return _orc.paccum_ex(self.mod_up(d, level), self.groups(level),
                              key_b, key_a, len(q), self.alpha, self.max_q,
                              self.offset(level), q + self.aux, self.log_n)

    def caccum(self, acc, ct, level):
        """acc (L + alpha limbs) += MontMul(ToMont(P mod q_l), ct) on q"""
        q = self.q(level)
        pp = _orc.p_prod(q, self.aux)
        out = acc.copy()
        n = 1 << self.log_n
        for i, p in enumerate(q):
            t = mont_mul_vec(ct[i], np.full(n, pp[i], np.uint32), p)
            out[i] = ((out[i].astype(np.uint64) + t) % p).astype(np.uint32)
        return out

    def _down(self, src, src_primes, drop, dst_primes):
        pos = {p: i for i, p in enumerate(src_primes) if i not in set(drop)}
        dst_src = [pos.get(p, -1) for p in dst_primes]
        return _orc.mod_down_ex(src, src_primes, drop, dst_primes, dst_src,
                                self.log_n)

    def rescale_src(self, level):
        """limb indices of level's q primes that leave on Rescale to
        level - 1 (ModSwitch.cu:263-303)"""
        (m, t), (m2, t2) = self.np(level), self.np(level - 1)
        L = m + t
        if t - t2 > 0:
            assert m - m2 <= 0
            return list(range(t - t2))
        assert m - m2 > 0 and t - t2 <= 0
        return list(range(L - (m - m2), L))

    def mod_down(self, acc, level):
        q = self.q(level)
        L = len(q)
        return self._down(acc, q + self.aux, list(range(L, L + self.alpha)), q)

    def mod_down_and_rescale(self, acc, level):
        q = self.q(level)
        L = len(q)
        drop = self.rescale_src(level) + list(range(L, L + self.alpha))
        return self._down(acc, q + self.aux, drop, self.q(level - 1))

    def rescale(self, x, level):
        return self._down(x, self.q(level), self.rescale_src(level),
                          self.q(level - 1))

    # ------------------------------------------------------- compositions
    def hmult(self, b1, a1, b2, a2, key_b, key_a, level, rescale):
        q = self.q(level)
        bx, ax, rx = _orc.tensor(b1, a1, b2, a2, q, self.log_n)
        acc_b, acc_a = self.key_mult(rx, level, key_b, key_a)
        acc_b = self.caccum(acc_b, bx, level)
        acc_a = self.caccum(acc_a, ax, level)
        down = self.mod_down_and_rescale if rescale else self.mod_down
        return down(acc_b, level), down(acc_a, level)

    def mult_key(self, b, a, key_b, key_a, level):
        acc_b, acc_a = self.key_mult(a, level, key_b, key_a)
        acc_b = self.caccum(acc_b, b, level)
        return self.mod_down(acc_b, level), self.mod_down(acc_a, level)

    def hrot(self, b, a, key_b, key_a, level, rot):
        mb, ma = self.mult_key(b, a, key_b, key_a, level)
        g = _orc.lib.orc_galois_factor(rot, self.log_n)
        return _orc.permute(mb, self.log_n, g), _orc.permute(ma, self.log_n, g)
