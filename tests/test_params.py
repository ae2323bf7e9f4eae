"""CPU tests of the JSON parameter loader against the reference's own
parameter files (copied as fixtures into tests/golden/params/ from the
reference's parameters/ directory): the layout of unittest/Testbed.h:95-179,
the level -> prime-count mapping, and clear errors for what this build does
not take (64-bit primes) or for malformed files."""
import json
import os

import pytest

PARAMS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "params")


def _text(name):
    return open(os.path.join(PARAMS, name)).read()


@pytest.fixture(scope="module")
def chd():
    import cheddar_amd
    return cheddar_amd


def test_bootparam_30_loads_with_its_level_map(chd):
    text = _text("bootparam_30.json")
    d = json.loads(text)
    p = chd.Param.from_json(text)
    assert p.max_level == len(d["level_config"]) - 1 == 34
    assert p.alpha == len(d["auxiliary_primes"]) == 12
    assert p.evk_limbs == 48 + 12
    for level, (main, ter) in enumerate(d["level_config"]):
        assert p.num_q(level) == main + ter


@pytest.mark.parametrize("name", ["bootparam_35.json", "bootparam_40.json"])
def test_terminal_prime_sets_load(chd, name):
    text = _text(name)
    d = json.loads(text)
    p = chd.Param.from_json(text)
    assert p.max_level == len(d["level_config"]) - 1
    assert p.evk_limbs == (len(d["main_primes"]) + len(d["terminal_primes"])
                           + len(d["auxiliary_primes"]))
    for level, (main, ter) in enumerate(d["level_config"]):
        assert p.num_q(level) == main + ter


def test_64bit_set_is_rejected_with_a_reason(chd):
    with pytest.raises(chd.ChdError, match="32-bit word"):
        chd.Param.from_json(_text("bootparam_40_64bit.json"))


@pytest.mark.parametrize("mutate,match", [
    (lambda d: d.pop("main_primes"), "Missing main_primes"),
    (lambda d: d.update(log_degree="16"), "log_degree should be an integer"),
    (lambda d: d.update(level_config=[[1, 0, 2]]), "array of pairs"),
    (lambda d: d.update(main_primes=[786433, 786435]), "NTT-friendly"),
])
def test_malformed_files_are_rejected(chd, mutate, match):
    d = json.loads(_text("bootparam_30.json"))
    mutate(d)
    with pytest.raises(chd.ChdError, match=match):
        chd.Param.from_json(json.dumps(d))


@pytest.mark.parametrize("log_degree", [12, 15, 17])
def test_degrees_other_than_2_16_are_rejected(chd, log_degree):
    """the reference documents only log_degree 16 (Parameter.h:33); every
    kernel here is built for N = 2^16, so another degree is refused with a
    reason instead of running wrong (its primes stay NTT-friendly for it)"""
    d = json.loads(_text("bootparam_30.json"))
    d["log_degree"] = log_degree
    with pytest.raises(chd.ChdError, match="only log_degree 16"):
        chd.Param.from_json(json.dumps(d))


def test_syntax_error_is_reported(chd):
    with pytest.raises(chd.ChdError, match="JSON"):
        chd.Param.from_json('{"log_degree": 16,')
