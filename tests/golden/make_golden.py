"""Writes tests/golden/ref_constants.json from oracle/_ref/refcheck.

refcheck is compiled (oracle/Makefile target `ref`) from the reference's own
host-only headers (include/common/PrimeUtils.h, CommonUtils.h). The fixture
holds its outputs: per-prime generator, psi, q^-1 mod 2^32, N^-1, R^2,
sampled Montgomery twiddles, and ModSwitch tables for two prime sets.
Run in a container that has /root/reference:  python tests/golden/make_golden.py
"""
import json
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "cheddar-fhe_amd", "python"))
from chd_primes import ntt_primes  # noqa: E402

REFCHECK = os.path.join(ROOT, "oracle", "_ref", "refcheck")

# (log_n, src primes, dst primes): a ModUp group at config-4 shape and the
# merged ModDown+Rescale source set {q_top} U P.
CASES = [
    (16, ntt_primes(30, 8), ntt_primes(30, 16, skip=8) + ntt_primes(31, 8)),
    (16, ntt_primes(30, 1, skip=23) + ntt_primes(31, 8), ntt_primes(30, 23)),
    (12, ntt_primes(31, 2, skip=8), ntt_primes(30, 3)),
]


def parse(text):
    out = {"primes": [], "tw": []}
    for line in text.splitlines():
        f = line.split()
        if f[0] == "prime":
            out["primes"].append([int(v) for v in f[1:]])
        elif f[0] == "tw":
            out["tw"].append([int(v) for v in f[1:]])
        else:
            out[f[0]] = [int(v) for v in f[1:]]
    return out


def run_case(log_n, src, dst):
    args = [REFCHECK, str(log_n), str(len(src)), str(len(dst))]
    args += [str(p) for p in src + dst]
    res = parse(subprocess.check_output(args, text=True))
    res.update(log_n=log_n, src=src, dst=dst)
    return res


def main():
    subprocess.check_call(["make", "-s", "-C", os.path.join(ROOT, "oracle"),
                           "ref"])
    cases = [run_case(*c) for c in CASES]
    with open(os.path.join(HERE, "ref_constants.json"), "w") as f:
        json.dump({"generator": "tests/golden/make_golden.py",
                   "twiddle_index": [0, 1, 2, 3, 5, 255, 256, 4097,
                                     "n/2+7", "n-1"],
                   "cases": cases}, f)


if __name__ == "__main__":
    main()
