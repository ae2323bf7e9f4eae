"""CPU check of the BConv table packing (chd_bconv_table_pack) and of the
kernel's data flow on it: the int8 MFMA operands are formed lane by lane in
the layouts the kernel uses (A: row = lane % 16, K = 16 (lane / 16) + byte;
B: column = lane % 16, same K; D: column = lane % 16, rows 4 (lane / 16) +
0..3), multiplied exactly in numpy, recombined as the kernel does (planes
paired in int32, joined in 64 bits, one signed Montgomery reduction, made
canonical) and compared with the oracle's BConv (ModSwitch.cu:23-171). The
shapes cover full, partial and packed last destination tiles (a job with at
most 8 sources whose last tile holds 1..8 destinations carries both
coefficient groups of a wave in the two K halves)."""
import ctypes

import numpy as np
import pytest

import _orc
from chd_primes import ntt_primes

LOG_N = 16
N = 1 << LOG_N
Q30 = ntt_primes(30, 32)
Q31 = ntt_primes(31, 48)


@pytest.fixture(scope="module")
def lib():
    import cheddar_amd
    lib = cheddar_amd.lib
    lib.chd_bconv_table_size.restype = ctypes.c_longlong
    lib.chd_bconv_table_size.argtypes = [ctypes.c_int, ctypes.c_int]
    lib.chd_bconv_table_pack.restype = ctypes.c_int
    lib.chd_bconv_table_pack.argtypes = [
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
        ctypes.c_int]
    return lib


def packed_table(lib, table, dst_primes):
    dst_len, src_len = table.shape
    size = lib.chd_bconv_table_size(src_len, dst_len)
    out = np.zeros(size, np.int8)
    t = np.ascontiguousarray(table, np.int32)
    d = np.ascontiguousarray(dst_primes, np.uint32)
    assert lib.chd_bconv_table_pack(out.ctypes.data, t.ctypes.data,
                                    d.ctypes.data, src_len, dst_len) == 0
    return out


def digits(c):
    """the kernel's signed byte digits of centred int32 values, as int8 x 4"""
    w = ((c.astype(np.int64) + 0x808080) & 0xFFFFFFFF) ^ 0x808080
    return w.astype(np.uint32).view(np.uint8).reshape(c.shape + (4,)).astype(
        np.int8)


def mont_reduce_lazy(y, p, pinv):
    """Basic.cuh:72-88 on int64 numpy arrays (|y| < p 2^31)"""
    y = y.astype(np.int64)
    lo = (y & 0xFFFFFFFF).astype(np.uint64)
    hi = y >> 32
    t = (lo * np.uint64(pinv & 0xFFFFFFFF)) & np.uint64(0xFFFFFFFF)
    t = t.astype(np.int64)
    t = np.where(t >= 1 << 31, t - (1 << 32), t)
    u = (t * np.int64(p)) >> 32
    return hi - u


def emulate_wave(table8, src, n0, src_len, dst_len, dst_primes):
    """outputs [dst_len][32] of the wave whose coefficients are n0 .. n0+31"""
    tiles = (dst_len + 15) // 16
    narrow = src_len <= 8
    rem = dst_len % 16
    packed = narrow and 0 < rem <= 8
    nk = (src_len + 15) // 16
    lanes = np.arange(64)
    r, g = lanes % 16, lanes // 16
    # A operands per K chunk and coefficient tile, 16 int8 per lane (4
    # sources x 4 digits): lane (r, g) holds sources i = 16 ch + 4 g + j of
    # coefficient n0 + 16 mt + r; with at most 8 sources, chunk 0's lanes
    # g >= 2 hold sources 4 (g & 1) + j of the second coefficient tile
    a = {}
    for ch in range(nk):
        for mt in range(2):
            byts = np.zeros((64, 16), np.int8)
            for lane in range(64):
                second = ch == 0 and narrow and g[lane] >= 2
                n = n0 + (16 if (mt == 1 or second) else 0) + r[lane]
                for j in range(4):
                    i = 4 * (g[lane] & 1) + j if (ch == 0 and narrow) else \
                        16 * ch + 4 * g[lane] + j
                    c = src[i, n] if i < src_len else 0
                    byts[lane, 4 * j:4 * j + 4] = digits(np.array([c]))[0]
            a[ch, mt] = byts
    planes = table8.reshape(tiles, nk, 4, 64, 16)
    out = np.zeros((dst_len, 32), np.uint32)

    def matrix(lane_bytes):
        # lane (row/column = lane % 16, K = 16 (lane / 16) + byte)
        m = np.zeros((16, 64), np.int64)
        for lane in range(64):
            m[lane % 16, 16 * (lane // 16):16 * (lane // 16) + 16] = \
                lane_bytes[lane]
        return m

    def finish(dplanes, col_to_dst, col_to_group):
        # D[row][col]: lane (col, g) holds rows 4 g .. 4 g + 3
        lo = dplanes[0] + 256 * dplanes[1]
        hi = dplanes[2] + 256 * dplanes[3]
        assert np.abs(lo).max() < 1 << 30 and np.abs(hi).max() < 1 << 30
        y = hi * 65536 + lo
        for col in range(16):
            k = col_to_dst(col)
            if k >= dst_len:
                continue
            p = int(dst_primes[k])
            pinv = int(_orc.lib.orc_inv_mod_base(p))
            u = mont_reduce_lazy(y[:, col], p, pinv)
            assert np.abs(u).max() < p
            u = np.where(u < 0, u + p, u)
            out[k, 16 * col_to_group(col) + np.arange(16)] = u

    regular = tiles - 1 if packed else tiles
    for tt in range(regular):
        for mt in range(2):
            d = [sum(matrix(a[ch, mt]) @ matrix(planes[tt, ch, pl]).T
                     for ch in range(nk)) for pl in range(4)]
            finish(d, lambda col, tt=tt: 16 * tt + col,
                   lambda col, mt=mt: mt)
    if packed:
        tt = tiles - 1
        d = [matrix(a[0, 0]) @ matrix(planes[tt, 0, pl]).T for pl in range(4)]
        finish(d, lambda col: 16 * tt + (col & 7), lambda col: col >> 3)
    return out


@pytest.mark.parametrize("src_len,dst_len", [
    (8, 40), (8, 24), (5, 23), (8, 8), (3, 5), (8, 17), (9, 24), (16, 8),
    (17, 24)])
def test_packing_and_operand_layouts(lib, src_len, dst_len):
    src_p = (Q30 + Q31)[:src_len]
    dst_p = Q31[16:16 + dst_len] if src_len > 8 else Q31[:dst_len]
    _, table = _orc.modswitch_consts(src_p, dst_p, LOG_N)
    table8 = packed_table(lib, table, dst_p)
    rng = np.random.default_rng(7 * src_len + dst_len)
    src = np.stack([rng.integers(-((p - 1) // 2), (p - 1) // 2 + 1, N)
                    .astype(np.int32) for p in src_p])
    src[:, :32] = np.array([(p - 1) // 2 for p in src_p], np.int32)[:, None]
    src[:, 32:64] = -src[:, :32]
    want = _orc.bconv(src, table, dst_p, LOG_N)
    for n0 in (0, 32, 4096 + 64, N - 32):
        got = emulate_wave(table8, src, n0, src_len, dst_len,
                           np.array(dst_p, np.uint32))
        assert np.array_equal(got, want[:, n0:n0 + 32]), (src_len, dst_len,
                                                           n0)
