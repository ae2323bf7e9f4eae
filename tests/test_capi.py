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
