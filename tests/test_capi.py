"""CPU tests of the C-ABI library: it loads, exports every function the
headers in include/ declare, and rejects invalid input with a status and a
message before touching the device (no compute call is made here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h)
           for h in ("cheddar_amd.h", "cheddar_kernels.h")]


def declared_functions():
    names = set()
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(chd_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return sorted(names)


@pytest.fixture(scope="module")
def chd():
    import cheddar_amd
    return cheddar_amd


def test_exports_every_declared_symbol(chd):
    names = declared_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(chd.lib, n)]
    assert not missing, missing


def test_version(chd):
    assert b"gfx950" in chd.lib.chd_version()


def test_ntt_plan_rejects_bad_prime(chd):
    with pytest.raises(chd.ChdError, match="NTT-friendly"):
        chd.NttPlan([1073479681 + 2])          # not 1 mod 2^17


def test_ntt_plan_rejects_large_prime(chd):
    with pytest.raises(chd.ChdError):
        chd.NttPlan([(1 << 31) + (1 << 17) + 1])


def test_param_validation(chd):
    from chd_primes import ntt_primes
    main = ntt_primes(30, 4)
    aux = ntt_primes(31, 2)
    with pytest.raises(chd.ChdError, match="NTT-friendly"):
        chd.Param(main[:3] + [main[3] + 2], aux, [(i, 0) for i in range(1, 5)])
    with pytest.raises(chd.ChdError, match="level"):
        chd.Param(main, aux, [(2, 0), (1, 0), (4, 0)])
    with pytest.raises(chd.ChdError, match="last level"):
        chd.Param(main, aux, [(1, 0), (2, 0)])


def test_null_arguments_return_status(chd):
    st = chd.lib.chd_ntt_forward(None, None, None, 1, 1, 0, None)
    assert st == -1
    assert b"invalid argument" in chd.lib.chd_last_error()
    st = chd.lib.chd_hmult(None, 0, None, None, None, None, None, None, None,
                           None, 0, 1, None)
    assert st == -1
    st = chd.lib.chd_bconv_apply(None, None, None, None)
    assert st == -1
    t = ctypes.c_void_p()
    st = chd.lib.chd_bconv_plan_create(ctypes.byref(t), 16, None, 0, None, 0)
    assert st == -1


# ---- argument checks of the batched kernel entry points (host side only:
# every call below is rejected before anything is launched)
P = ctypes.c_void_p


class Tables(ctypes.Structure):
    _fields_ = [(n, P) for n in ("q", "qinv", "tw", "itw", "twist")]


class LimbMap(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("num_q", "skip_lo", "skip_len",
                                            "src_gap", "tab_off", "tab_gap",
                                            "cst_gap")]


class GsWideArgs(ctypes.Structure):
    _fields_ = [("num_bs", ctypes.c_int), ("num_gs", ctypes.c_int),
                ("add_to_dst", ctypes.c_int), ("pt_stride", ctypes.c_int),
                ("bs_b", P * 32), ("bs_a", P * 32), ("pt_table", P),
                ("dst_b", P * 32), ("dst_a", P * 32), ("pt_tiled", P),
                ("tiled_rows", ctypes.c_int)]


FAKE = P(0x1000)  # never dereferenced: the calls fail their checks first


def _kernel_lib(chd):
    lib = chd.lib
    lib.chd_k_gs_fused_wide.argtypes = [ctypes.POINTER(Tables),
                                        ctypes.POINTER(LimbMap),
                                        ctypes.POINTER(GsWideArgs),
                                        ctypes.c_int, P]
    lib.chd_k_modup_keyacc_batch.argtypes = [ctypes.POINTER(Tables), P,
                                             ctypes.c_int, P]
    lib.chd_k_ntt_fwd_groups_batch.argtypes = [
        ctypes.POINTER(Tables), ctypes.POINTER(LimbMap), P, ctypes.c_longlong,
        ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
        ctypes.c_int, P]
    lib.chd_k_ntt_fwd_moddown_multi.argtypes = [
        ctypes.POINTER(Tables), ctypes.POINTER(LimbMap), ctypes.POINTER(P),
        ctypes.c_int, ctypes.c_int, P, ctypes.c_longlong, P,
        ctypes.c_longlong, ctypes.c_int, ctypes.c_int, P, P, P]
    lib.chd_k_ntt_fwd_moddown_bconv1_multi.argtypes = [
        ctypes.POINTER(Tables), ctypes.POINTER(LimbMap), ctypes.POINTER(P),
        ctypes.c_int, ctypes.c_int, P, ctypes.c_longlong, P, P,
        ctypes.c_longlong, ctypes.c_int, ctypes.c_int, P, P, P]
    lib.chd_k_ntt_fwd_moddown.argtypes = [
        ctypes.POINTER(Tables), ctypes.POINTER(LimbMap), P, ctypes.c_int, P,
        ctypes.c_int, ctypes.c_int, P, P, P]
    return lib


def test_ntt_inv_single_pass_checks(chd):
    """chd_k_ntt_inv_1p refuses an overlapping destination and tables
    without the twist table, before any launch"""
    lib = chd.lib
    lib.chd_k_ntt_inv_1p.argtypes = [
        ctypes.POINTER(Tables), ctypes.POINTER(LimbMap), P, ctypes.c_longlong,
        P, ctypes.c_longlong, ctypes.c_int, ctypes.c_int, P, ctypes.c_int, P]
    m = LimbMap(num_q=32, skip_lo=1 << 30)
    ps = 32 << 16
    t = Tables(twist=FAKE)
    assert lib.chd_k_ntt_inv_1p(t, m, FAKE, ps, FAKE, ps, 32, 2, FAKE, 0,
                                None) == -1
    assert b"apart from the destination" in lib.chd_last_error()
    # half a limb apart: still overlapping
    assert lib.chd_k_ntt_inv_1p(t, m, P(0x1000 + 4 * (1 << 15)), ps, FAKE,
                                ps, 32, 2, FAKE, 0, None) == -1
    t = Tables()
    assert lib.chd_k_ntt_inv_1p(t, m, P(1 << 40), ps, FAKE, ps, 32, 2, FAKE,
                                0, None) == -1
    assert b"invalid argument" in lib.chd_last_error()


def test_gs_fused_wide_checks(chd):
    lib = _kernel_lib(chd)
    t, m = Tables(), LimbMap(num_q=20)
    a = GsWideArgs(num_bs=4, num_gs=12, pt_stride=4, pt_table=FAKE)
    for j in range(4):
        a.bs_b[j] = a.bs_a[j] = FAKE
    for g in range(32):
        a.dst_b[g] = a.dst_a[g] = FAKE
    # giant steps must be padded to 8, 16, 24, 28 or 32
    assert lib.chd_k_gs_fused_wide(t, m, a, 28, None) == -1
    assert b"num_gs" in chd.lib.chd_last_error()
    # baby steps come in fours
    a.num_gs, a.num_bs = 16, 3
    assert lib.chd_k_gs_fused_wide(t, m, a, 28, None) == -1
    a.num_bs, a.pt_table = 4, None
    assert lib.chd_k_gs_fused_wide(t, m, a, 28, None) == -1


def test_gs_tiled_copy_checks(chd):
    lib = chd.lib
    lib.chd_k_gs_pack_tiled.argtypes = [P, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, P, P]
    lib.chd_k_gs_untile_row.argtypes = [P, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, P, P]
    # rows in [1, 32], stride in [1, 32], pointers given
    for rows, stride, tab, dst in ((0, 4, FAKE, FAKE), (33, 4, FAKE, FAKE),
                                   (2, 0, FAKE, FAKE), (2, 33, FAKE, FAKE),
                                   (2, 4, None, FAKE), (2, 4, FAKE, None)):
        assert lib.chd_k_gs_pack_tiled(tab, rows, stride, 28, dst, None) == -1
        assert b"chd_k_gs_pack_tiled" in lib.chd_last_error()
    # the row inside the array, no more limbs out than it holds
    for g, dl in ((-1, 4), (2, 4), (0, 29), (0, -1)):
        assert lib.chd_k_gs_untile_row(FAKE, 2, 4, 28, g, dl, FAKE,
                                       None) == -1
        assert b"chd_k_gs_untile_row" in lib.chd_last_error()
    # a tiled array with more rows than the launch computes is refused
    a = GsWideArgs(num_bs=4, num_gs=16, pt_stride=4, pt_table=FAKE,
                   pt_tiled=FAKE, tiled_rows=17)
    for j in range(4):
        a.bs_b[j] = a.bs_a[j] = FAKE
    for g in range(32):
        a.dst_b[g] = a.dst_a[g] = FAKE
    k = _kernel_lib(chd)
    t, m = Tables(), LimbMap(num_q=20)
    assert k.chd_k_gs_fused_wide(t, m, a, 28, None) == -1
    assert b"tiled_rows" in chd.lib.chd_last_error()


def test_batched_entry_points_reject_bad_counts(chd):
    lib = _kernel_lib(chd)
    t, m = Tables(), LimbMap(num_q=20, skip_lo=1 << 30)
    # more key accumulations than one launch takes, or none
    assert lib.chd_k_modup_keyacc_batch(t, FAKE, 9, None) == -1
    assert lib.chd_k_modup_keyacc_batch(t, FAKE, 0, None) == -1
    # ModUp column passes of too many inputs
    assert lib.chd_k_ntt_fwd_groups_batch(t, m, FAKE, 1 << 20, 3, 9, 8, 0,
                                          28, 0, None) == -1


def test_moddown_ntt_rejects_overlapping_source(chd):
    lib = _kernel_lib(chd)
    t, m = Tables(), LimbMap(num_q=20, skip_lo=1 << 30)
    n = 1 << 16
    base = 0x10000000
    dst = (P * 2)(P(base), P(base + 40 * 4 * n))
    # the source starts inside dst[1]: the single-pass NTT cannot run
    src = P(base + 45 * 4 * n)
    st = lib.chd_k_ntt_fwd_moddown_multi(t, m, dst, 2, 20, src, 20 * n, None,
                                         0, 0, 0, FAKE, None, None)
    assert st == -1
    assert b"overlaps" in chd.lib.chd_last_error()


def test_moddown_ntt_rejects_overlapping_src2(chd):
    """the epilogue operand src2 may not overlap any destination, also when
    it starts between two destination limbs rather than on one"""
    lib = _kernel_lib(chd)
    t, m = Tables(), LimbMap(num_q=20, skip_lo=1 << 30)
    n = 1 << 16
    base = 0x10000000
    dst = (P * 2)(P(base), P(base + 40 * 4 * n))
    src = P(base + 100 * 4 * n)            # disjoint from both
    for src2 in (P(base + 45 * 4 * n),     # inside dst[1]
                 P(base + 39 * 4 * n)):    # runs from dst[0]'s gap into dst[1]
        st = lib.chd_k_ntt_fwd_moddown_multi(t, m, dst, 2, 20, src, 20 * n,
                                             src2, 20 * n, 0, 20, FAKE, None,
                                             None)
        assert st == -1
        assert b"src2 overlaps" in chd.lib.chd_last_error()
    st = lib.chd_k_ntt_fwd_moddown(t, m, P(base), 20, P(base + 19 * 4 * n),
                                   0, 20, FAKE, None, None)
    assert st == -1
    assert b"src2 overlaps" in chd.lib.chd_last_error()


def test_moddown_ntt_checks_each_polynomial_of_a_descending_source(chd):
    """polynomials of src and src2 may be any distance apart, also below
    the first one (a negative stride, as when a ciphertext's ax sits below
    its bx): each polynomial is checked against every destination"""
    lib = _kernel_lib(chd)
    t, m = Tables(), LimbMap(num_q=20, skip_lo=1 << 30)
    n = 1 << 16
    base = 0x10000000
    dst = (P * 2)(P(base), P(base + 40 * 4 * n))
    # polynomial 1 of the source lands on dst[0]; polynomial 0 is clear
    st = lib.chd_k_ntt_fwd_moddown_multi(t, m, dst, 2, 20,
                                         P(base + 100 * 4 * n), -100 * n,
                                         None, 0, 0, 0, FAKE, None, None)
    assert st == -1
    assert b"source overlaps" in chd.lib.chd_last_error()
    # the same for the epilogue operand
    st = lib.chd_k_ntt_fwd_moddown_multi(t, m, dst, 2, 20,
                                         P(base + 100 * 4 * n), 20 * n,
                                         P(base + 200 * 4 * n), -165 * n, 0,
                                         20, FAKE, None, None)
    assert st == -1
    assert b"src2 overlaps" in chd.lib.chd_last_error()


def test_moddown_bconv1_ntt_checks(chd):
    """the one-source ModDown NTT reads its source limb of each polynomial
    while other workgroups write: a source limb inside a destination, a
    src2 limb inside a destination and missing operands are rejected
    before any launch"""
    lib = _kernel_lib(chd)
    t, m = Tables(), LimbMap(num_q=20, skip_lo=1 << 30)
    n = 1 << 16
    base = 0x10000000
    dst = (P * 2)(P(base), P(base + 40 * 4 * n))
    f = lib.chd_k_ntt_fwd_moddown_bconv1_multi
    # polynomial 1's source limb (stride -60 limbs) is dst[1]'s limb 5
    st = f(t, m, dst, 2, 20, P(base + 105 * 4 * n), -60 * n, FAKE, None, 0,
           0, 0, FAKE, None, None)
    assert st == -1
    assert b"source overlaps" in chd.lib.chd_last_error()
    st = f(t, m, dst, 2, 20, P(base + 100 * 4 * n), n, FAKE,
           P(base + 30 * 4 * n), 20 * n, 0, 20, FAKE, None, None)
    assert st == -1
    assert b"src2 overlaps" in chd.lib.chd_last_error()
    for src1, table in ((None, FAKE), (P(base + 100 * 4 * n), None)):
        st = f(t, m, dst, 2, 20, src1, n, table, None, 0, 0, 0, FAKE, None,
               None)
        assert st == -1
        assert b"invalid argument" in chd.lib.chd_last_error()


def test_forward_ntt_rejects_partial_overlap(chd):
    """the forward NTT runs in place (two passes) or out of place into
    disjoint memory; any other overlap would race between workgroups and is
    rejected before a launch: a shifted destination, the same base with
    another polynomial stride, and an in-place call whose source has a gap"""
    lib = chd.lib
    lib.chd_k_ntt_fwd.argtypes = [ctypes.POINTER(Tables),
                                  ctypes.POINTER(LimbMap), P,
                                  ctypes.c_longlong, P, ctypes.c_longlong,
                                  ctypes.c_int, ctypes.c_int, P, P]
    t, m = Tables(), LimbMap(num_q=20, skip_lo=1 << 30)
    n = 1 << 16
    base = 0x10000000
    cases = [
        (P(base + 3 * 4 * n), 20 * n, P(base), 20 * n, 1, m),
        (P(base), 24 * n, P(base), 20 * n, 2, m),
        (P(base), 20 * n, P(base), 20 * n, 1,
         LimbMap(num_q=16, skip_lo=1 << 30, src_gap=4)),
    ]
    lib.chd_k_ntt_fwd_2p.argtypes = lib.chd_k_ntt_fwd.argtypes
    for fn in (lib.chd_k_ntt_fwd, lib.chd_k_ntt_fwd_2p):
        for dst, dps, src, sps, polys, mm in cases:
            st = fn(t, mm, dst, dps, src, sps, 20, polys, None, None)
            assert st == -1
            assert b"overlap" in chd.lib.chd_last_error()


def test_binding_handles_released_cleanly_at_exit():
    """handles still alive at interpreter exit are destroyed through the
    function bound when they were made, not through module globals that
    exit has already cleared: nothing is printed to stderr"""
    import subprocess
    import sys
    code = (
        "import sys\n"
        "sys.path.insert(0, %r)\n"
        "sys.path.insert(0, %r)\n"
        "import cheddar_amd\n"
        "from gpu_util import config4\n"
        "main, aux, levels = config4()\n"
        "keep = [cheddar_amd.Param(main, aux, levels) for _ in range(3)]\n"
        % (os.path.join(ROOT, "cheddar-fhe_amd", "python"),
           os.path.join(ROOT, "tests")))
    res = subprocess.run([sys.executable, "-c", code], capture_output=True,
                         text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    assert res.stderr.strip() == "", res.stderr
