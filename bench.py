"""Benchmark of the MI355X CKKS key-switch hot path.

Headline (BASELINE.json "metric", configs[1]): batched NTT + INTT of one
ciphertext, 2 polynomials x 32 RNS limbs, N = 2^16, 32 distinct 30-bit
primes = 1 mod 2^17, limb-major. One step = forward NTT of all 64 limbs
followed by the inverse NTT (128 limb-transforms). value = limb-transforms/s
with inputs resident in HBM; the input/output buffers rotate over a set
larger than the 256 MB MALL so the timed traffic comes from HBM.

The same JSON line carries the other two parts of the metric: the HMult
key-switch time at config 4 (L = 24, dnum = 3, alpha = 8, merged
ModDown+Rescale) and the config-3 BConv time, both measured with HIP events,
the time of a config-5-shaped hoisted BSGS linear transform, plus the
roofline of the NTT and the CPU baseline (the oracle's scalar Montgomery NTT
on this host, bounded sample).

    python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "cheddar-fhe_amd", "python"))

HBM_PEAK_GBS = 8000.0
N = 1 << 16
LIMB_BYTES = 4 * N
# one limb-transform moves one limb in and one limb out (algorithmic bytes)
LIMB_TRANSFORM_BYTES = 2 * LIMB_BYTES
MALL_BYTES = 256 << 20
# calibration copy: 1 GiB each way, far beyond L2 and the 256 MiB MALL
COPY_BYTES = 1 << 30


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true",
                    help="skip the CPU-baseline leg")
    ap.add_argument("--only", choices=["ntt_fwd", "ntt_inv", "hmult",
                                       "bconv", "copy", "hoist"],
                    help="run only this workload's timed loop (for "
                         "profiling); prints its average time")
    return ap.parse_args()


def event_time_ms(fn, iters, stream):
    import torch
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(iters):
        fn(i)
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end)


def bench_ntt(chd, steps, warmup):
    import numpy as np
    import torch
    from chd_primes import ntt_primes
    primes = ntt_primes(30, 32)
    plan = chd.NttPlan(primes)
    set_bytes = 2 * 32 * LIMB_BYTES
    nsets = max(4, (2 * MALL_BYTES) // set_bytes + 1)  # > 2x MALL per role
    rng = np.random.default_rng(0xC0FFEE02)
    host = np.stack([np.stack([rng.integers(0, p, N, dtype=np.uint64)
                               for p in primes]) for _ in range(2)])
    base = torch.from_numpy(host.astype(np.uint32).view(np.int32)).cuda()
    srcs = [base.clone() for _ in range(nsets)]
    dsts = [torch.empty_like(base) for _ in range(nsets)]
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)

    def step(i):
        s, d = srcs[i % nsets], dsts[i % nsets]
        plan.forward(d, s, 32, 2, stream=sp)
        plan.inverse(s, d, 32, 2, mont_conv=False, stream=sp)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    ms = event_time_ms(step, steps, stream)
    torch.cuda.synchronize()
    # the inverse with mont_conv=False returns the input: check it stayed put
    ok = all(torch.equal(srcs[i], base) for i in range(nsets))
    # forward-only timing for the roofline (both passes of one direction)
    def fwd(i):
        plan.forward(dsts[i % nsets], srcs[i % nsets], 32, 2, stream=sp)
    fwd_ms = event_time_ms(fwd, steps, stream) / steps
    inv_ms = event_time_ms(
        lambda i: plan.inverse(srcs[i % nsets], dsts[i % nsets], 32, 2,
                               mont_conv=False, stream=sp), steps,
        stream) / steps
    # warm (MALL-resident) figure on one buffer set
    warm_ms = event_time_ms(lambda i: plan.forward(dsts[0], srcs[0], 32, 2,
                                                   stream=sp), steps,
                            stream) / steps
    return ms, fwd_ms, inv_ms, warm_ms, ok


def bench_hmult(chd, iters=20):
    import numpy as np
    import torch
    from chd_primes import ntt_primes
    main, aux = ntt_primes(30, 24), ntt_primes(31, 8)
    param = chd.Param(main, aux, [(i, 0) for i in range(1, 25)])
    ctx = chd.Context(param)
    rng = np.random.default_rng(0xC0FFEE04)

    def limbs(primes):
        a = np.stack([rng.integers(0, p, N, dtype=np.uint64) for p in primes])
        return torch.from_numpy(a.astype(np.uint32).view(np.int32)).cuda()
    a = (limbs(main), limbs(main))
    b = (limbs(main), limbs(main))
    kb = [limbs(main + aux) for _ in range(3)]
    ka = [limbs(main + aux) for _ in range(3)]
    res = (torch.empty(23, N, dtype=torch.int32, device="cuda"),
           torch.empty(23, N, dtype=torch.int32, device="cuda"))
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)

    def run(_):
        ctx.hmult(23, res, a, b, kb, ka, rescale=True, stream=sp)
    for _ in range(3):
        run(0)
    torch.cuda.synchronize()
    return event_time_ms(run, iters, stream) / iters


def bench_hoist(chd, iters=5):
    """config 5's shape: a 768 x 768 BSGS linear transform (28 baby steps,
    28 giant steps, 768 diagonal plaintexts) on one ciphertext at L = 20 of
    the config-4 chain, double hoisting. Residues are synthetic uniform
    values below every prime (the plaintexts are not encoder output)."""
    import torch
    from chd_primes import ntt_primes
    main, aux = ntt_primes(30, 24), ntt_primes(31, 8)
    param = chd.Param(main, aux, [(i, 0) for i in range(1, 25)])
    ctx = chd.Context(param)
    L, level = 20, 19
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0xC0FFEE05)

    def limbs(n):
        return torch.randint(0, 1 << 29, (n, N), dtype=torch.int32,
                             device="cuda", generator=gen)
    bs = list(range(28))
    gs = [28 * k for k in range(28)]
    pts = {(g, b): limbs(L + 8) for g in gs for b in bs if g + b < 768}
    rots = sorted(set(bs[1:] + gs[1:]))
    keys = {r: ([limbs(32) for _ in range(3)], [limbs(32) for _ in range(3)])
            for r in rots}
    h = chd.Hoist(ctx, level, gs, bs, pts)
    del pts
    ct = (limbs(L), limbs(L))
    res = (torch.empty(L - 1, N, dtype=torch.int32, device="cuda"),
           torch.empty(L - 1, N, dtype=torch.int32, device="cuda"))
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    for _ in range(2):
        h.run(res, ct, keys, stream=sp)
    torch.cuda.synchronize()
    return event_time_ms(lambda i: h.run(res, ct, keys, stream=sp), iters,
                         stream) / iters


def bench_bconv(chd, iters=50):
    import numpy as np
    import torch
    from chd_primes import ntt_primes
    src_p, dst_p = ntt_primes(30, 8), ntt_primes(31, 40)
    plan = chd.BconvPlan(src_p, dst_p)
    rng = np.random.default_rng(0xC0FFEE03)
    x = np.stack([rng.integers(-((p - 1) // 2), (p - 1) // 2 + 1, N)
                  for p in src_p]).astype(np.int32)
    src = torch.from_numpy(x).cuda()
    dst = torch.empty(40, N, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    for _ in range(3):
        plan.apply(dst, src, stream=sp)
    torch.cuda.synchronize()
    return event_time_ms(lambda i: plan.apply(dst, src, stream=sp), iters,
                         stream) / iters


def cpu_baseline(seconds=10.0):
    """Oracle's scalar Montgomery NTT + INTT (1 thread) on a bounded sample
    of the config-2 workload: repeated 8-limb batches for ~`seconds`."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import _orc  # the checker library, timed here only as the CPU baseline
    from chd_primes import ntt_primes
    primes = ntt_primes(30, 32)[:8]
    rng = np.random.default_rng(0xC0FFEE02)
    x = np.stack([rng.integers(0, p, N, dtype=np.uint64)
                  for p in primes]).astype(np.uint32).reshape(-1)
    _orc.lib.orc_set_threads(1)
    pr = _orc.u32(primes)
    _orc.lib.orc_ntt_batch(x, 8, 16, pr, 0)   # warm the twiddle cache
    _orc.lib.orc_intt_batch(x, 8, 16, pr, 0)
    done, t0 = 0, time.perf_counter()
    while True:
        _orc.lib.orc_ntt_batch(x, 8, 16, pr, 0)
        _orc.lib.orc_intt_batch(x, 8, 16, pr, 0)
        done += 16
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"value": done / el, "unit": "limb-transforms/s", "cores": 1,
            "kind": "port",
            "sample": "%d limb-transforms (8-limb NTT+INTT batches of the "
                      "config-2 primes, N=2^16) in %.1f s, scalar C "
                      "Montgomery restatement, gcc -O2, 1 thread"
                      % (done, el)}


def run_only(chd, what, steps):
    """one workload's timed loop, for rocprofv3 runs"""
    import numpy as np
    import torch
    from chd_primes import ntt_primes
    if what == "hmult":
        return bench_hmult(chd, steps) * 1e3
    if what == "bconv":
        return bench_bconv(chd, steps) * 1e3
    if what == "hoist":
        return bench_hoist(chd, steps) * 1e3
    if what == "copy":
        # plain device copy of COPY_BYTES: the reference point that scales
        # the FETCH_SIZE / WRITE_SIZE counters into HBM bytes
        src = torch.ones(COPY_BYTES // 4, dtype=torch.int32, device="cuda")
        dst = torch.empty_like(src)
        stream = torch.cuda.current_stream()
        fn = lambda i: dst.copy_(src)  # noqa: E731
        fn(0)
        torch.cuda.synchronize()
        return event_time_ms(fn, steps, stream) / steps * 1e3
    primes = ntt_primes(30, 32)
    plan = chd.NttPlan(primes)
    rng = np.random.default_rng(0xC0FFEE02)
    host = np.stack([np.stack([rng.integers(0, p, N, dtype=np.uint64)
                               for p in primes]) for _ in range(2)])
    src = torch.from_numpy(host.astype(np.uint32).view(np.int32)).cuda()
    dst = torch.empty_like(src)
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    if what == "ntt_fwd":
        fn = lambda i: plan.forward(dst, src, 32, 2, stream=sp)  # noqa: E731
    else:
        fn = lambda i: plan.inverse(dst, src, 32, 2, stream=sp)  # noqa: E731
    fn(0)
    torch.cuda.synchronize()
    return event_time_ms(fn, steps, stream) / steps * 1e3


def traffic_from_profile():
    path = os.path.join(ROOT, "profiles", "ntt_fwd_config2_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("bytes_per_forward_ntt")


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py measures one GPU: every box in this run has one "
              "MI355X and the key-switch path is not sharded across GPUs "
              "(see DESIGN.md, 'More than one GPU'). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("no HIP device", file=sys.stderr)
        sys.exit(1)
    import cheddar_amd as chd

    if args.only:
        print(json.dumps({"only": args.only,
                          "us": run_only(chd, args.only, args.steps)}))
        return
    ms, fwd_ms, inv_ms, warm_ms, ok = bench_ntt(chd, args.steps, args.warmup)
    if not ok:
        print("NTT round trip changed the data", file=sys.stderr)
        sys.exit(1)
    lt = 128 * args.steps / (ms / 1e3)
    hmult_us = bench_hmult(chd) * 1e3
    bconv_us = bench_bconv(chd) * 1e3
    hoist_ms = bench_hoist(chd)
    fwd_bytes = 64 * LIMB_TRANSFORM_BYTES
    achieved = fwd_bytes / (fwd_ms / 1e3) / 1e9
    line = {
        "metric": "NTT limb-transforms/s @N=2^16; HMult keyswitch us; "
                  "% HBM/MFMA roofline",
        "value": lt,
        "unit": "limb-transforms/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32",
        "data": "synthetic (seeded uniform residues)",
        "config": {
            "workload": "config2: batched NTT+INTT of one ciphertext, 2 polys "
                        "x 32 limbs, N=2^16, 30-bit primes, limb-major, "
                        "buffers rotated over %d MiB" % 0,
            "limb_transforms_per_step": 128,
        },
        "roofline": {
            "kernel": "forward NTT (ntt_fwd_1p: single pass, one launch, "
                      "four workgroups per limb)",
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic_from_profile(),
        },
        "extra": {
            "ntt_forward_us": fwd_ms * 1e3,
            "ntt_inverse_us": inv_ms * 1e3,
            "ntt_forward_warm_mall_us": warm_ms * 1e3,
            "hmult_keyswitch_us_config4": hmult_us,
            "bconv_us_config3_warm": bconv_us,
            "hoist_bsgs_ms_config5_shape": hoist_ms,
            "notes": "hmult: warm (same key and inputs each step), host "
                     "enqueue included; hoist: 768x768 BSGS (28 baby, 28 "
                     "giant steps, 54 rotation keys, 768 plaintexts) at "
                     "L=20, synthetic plaintexts",
        },
    }
    nsets = max(4, (2 * MALL_BYTES) // (2 * 32 * LIMB_BYTES) + 1)
    line["config"]["workload"] = line["config"]["workload"].replace(
        "%d MiB" % 0, "%d MiB" % (2 * nsets * 16))
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line))


if __name__ == "__main__":
    main()
