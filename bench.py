"""Benchmark of the fused-contraction hot path on one MI355X.

Headline (BASELINE.json metric, config 4): DF-MP2 correlation energy,
nocc=64 nvir=320 naux=1200, float64, inputs resident in HBM. One step = one
trntensor_amd.mp2_energy call. value = algorithmic GFLOP/s
(2080 occupied pairs i<=j x 2*nvir^2*naux = 5.112e11 FLOP per step).

Also measured in the same run (secondary fields of the one JSON line):
config 3 AO->MO half transform 'mi,mnP->inP' (GB/s and binding-roofline
fraction), config 4 in float32, config 2 GEMM/bmm with alpha/beta, config 1
einsum-loop latency, config 5 greedy path. The CPU baseline is the
reference's CPU path restated in oracle/cpu_ref.py, timed on the host on a
bounded sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extra] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK = {"f64": 78.6e12, "f32": 157.3e12, "bf16": 2.5e15, "hbm": 8.0e12}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # The GPU ramps its clocks over the first ~0.1-0.2 s of work after idle;
    # 25 warm-up steps (~0.2 s) put the timed steps in steady state.
    ap.add_argument("--warmup", type=int, default=25)
    ap.add_argument("--no-extra", action="store_true", help="headline only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default="", help="comma list of extra configs (c1,c2,c3,c4f32,c4naux,c5,f1,a5)")
    ap.add_argument("--skip-headline", action="store_true", help="run only the extra configs")
    ap.add_argument(
        "--calibrate-copy",
        action="store_true",
        help="only copy 1 GiB device-to-device 5 times (reference kernel for the HBM byte counters)",
    )
    return ap.parse_args()


def timed(torch, fn, steps, warmup):
    """(wall ms/step, mean event ms/step, median event ms/step). Events are
    recorded on torch's current stream, which is the stream the library
    launches on."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = time.perf_counter()
    for a, b in evs:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    times = [a.elapsed_time(b) for a, b in evs]
    return wall, statistics.mean(times), statistics.median(times)


def timed_steady(torch, fn, steps, min_warm_s=0.3):
    """(wall ms/step, median event ms/step) after warming up for at least
    `min_warm_s` seconds of work (the secondary configs follow host-side input
    generation, during which the GPU idles and its clocks drop)."""
    t0 = time.perf_counter()
    n = 0
    while n < 2 or time.perf_counter() - t0 < min_warm_s:
        fn()
        torch.cuda.synchronize()
        n += 1
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = time.perf_counter()
    for a, b in evs:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return wall, statistics.median(a.elapsed_time(b) for a, b in evs)


def measured_peaks(torch, dev):
    """Rates this device sustains in microbenchmarks: fp64/fp32/bf16 MFMA with no
    memory traffic (tt_mfma_rate_probe) and HBM streams with no arithmetic
    (tt_hbm_probe). The datasheet peaks assume the maximum clock; these are
    what the kernels' fractions can also be read against."""
    from trntensor_amd.hip import _lib

    lib = _lib.load()
    st = torch.cuda.current_stream(dev).cuda_stream
    wgs = 1024
    out = {}
    cases = (
        ("mfma_f64_TFLOPs", _lib.TT_F64, torch.float64, 20000, 2048),
        ("mfma_f32_TFLOPs", _lib.TT_F32, torch.float32, 40000, 2048),
        ("mfma_bf16_TFLOPs", _lib.TT_BF16, torch.bfloat16, 40000, 16384),
    )
    for key, code, dt, iters, flop_per_mfma in cases:
        buf = torch.empty(wgs, dtype=dt, device=dev)
        flop = wgs * 4 * iters * 8 * flop_per_mfma

        def run():
            _lib.check(lib.tt_mfma_rate_probe(code, wgs, iters, buf.data_ptr(), st), "tt_mfma_rate_probe")

        _, ms = timed_steady(torch, run, 10)
        out[key] = round(flop / (ms * 1e-3) / 1e12, 2)
    out.update(hbm_probe(torch, dev, lib, st))
    return out


def hbm_probe(torch, dev, lib, st, gib=4):
    """HBM rate from tt_hbm_probe: read-only, write-only and copy streams of
    `gib` GiB each (16x the 256 MB MALL), 16-byte accesses, non-temporal or
    through the caches, 1024/2048/4096 workgroups. hbm_GBps is the best of them (bytes read plus
    bytes written per second); every case is listed under hbm_probe."""
    from trntensor_amd.hip import _lib

    nbytes = gib << 30
    src = torch.ones(nbytes // 8, dtype=torch.float64, device=dev)
    dst = torch.empty_like(src)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    cases = {}
    for mode, name, moved in ((0, "read", nbytes), (1, "write", nbytes), (2, "copy", 2 * nbytes)):
        for cached in (0, 4):
            for wgs in (1024, 2048, 4096):
                def run(m=mode + cached, wgs=wgs):
                    _lib.check(lib.tt_hbm_probe(m, src.data_ptr(), dst.data_ptr(), nbytes, wgs, flag.data_ptr(), st),
                               "tt_hbm_probe")

                _, ms = timed_steady(torch, run, 10, 0.1)
                cases[f"{name}_{'cached' if cached else 'nt'}_wg{wgs}"] = round(moved / (ms * 1e-3) / 1e9, 1)
    del src, dst
    best = max(cases, key=cases.get)
    return {
        "hbm_GBps": cases[best],
        "hbm_method": f"tt_hbm_probe {best} on {gib} GiB buffers, 16-byte accesses, "
        "median of 10 HIP-event-timed launches",
        "hbm_probe": cases,
    }


def add_measured_fractions(extra, peaks):
    """Next to each datasheet fraction in the config results, the same achieved
    rate over the peak this device sustains in a microbenchmark
    (`measured_peaks`): key + "_of_measured". The dtype of a fraction comes
    from the nearest enclosing key naming one (f32, bf16; fp64 otherwise)."""
    ratio = {
        "f64": PEAK["f64"] / (peaks["mfma_f64_TFLOPs"] * 1e12),
        "f32": PEAK["f32"] / (peaks["mfma_f32_TFLOPs"] * 1e12),
        "bf16": PEAK["bf16"] / (peaks["mfma_bf16_TFLOPs"] * 1e12),
        "hbm": PEAK["hbm"] / (peaks["hbm_GBps"] * 1e9),
    }

    def dtype_of(name, inherited):
        for dt in ("bf16", "f32", "f64"):
            if dt in name:
                return dt
        return inherited

    over = []

    def put(d, key, value, path):
        d[key] = round(value, 4)
        if value > 1.0:
            over.append(f"{path}.{key}")

    def walk(d, dt, path):
        for k, v in list(d.items()):
            if isinstance(v, dict):
                if k != "cpu":
                    walk(v, dtype_of(k, dt), f"{path}.{k}" if path else k)
            elif isinstance(v, (int, float)) and not isinstance(v, bool):
                if k in ("frac_mfma", "frac_binding_roofline", "ao_to_mo_frac_mfma"):
                    put(d, k + "_of_measured", v * ratio[dt], path)
                elif k == "frac_mfma_f32":
                    put(d, k + "_of_measured", v * ratio["f32"], path)
                elif k == "frac_hbm":
                    put(d, k + "_of_measured", v * ratio["hbm"], path)

    walk(extra, "f64", "")
    # A fraction above 1 means the probe did not find the device's peak.
    return over


def host_info(torch):
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    found = re.search(r"BLAS_INFO=([^,\s]+)", torch.__config__.show())
    blas = found.group(1) if found else "unknown"
    return {"cpu_model": model, "logical_cpus": os.cpu_count(), "torch": torch.__version__, "blas": blas}


def mp2_inputs(torch, dtype, nocc=64, nvir=320, naux=1200):
    g = torch.Generator().manual_seed(0)
    B = torch.randn(nocc, nvir, naux, generator=g, dtype=torch.float64) * 0.05
    eo = torch.sort(-20 + 19.7 * torch.rand(nocc, generator=g, dtype=torch.float64))[0]
    ev = torch.sort(0.1 + 4.9 * torch.rand(nvir, generator=g, dtype=torch.float64))[0]
    return B.to(dtype), eo.to(dtype), ev.to(dtype)


TRAFFIC_FILE = "profiles/traffic.json"
PROFILE_FILE = "profiles/headline_profile.json"
# Sustained-clock spread between boxes of the pool under a long MFMA-bound
# load, as a fraction of the kernel time: the same build's headline measured
# 7.49-8.23 ms on different boxes while the MFMA-only probe read 77.3-78.0
# TFLOP/s on all of them.
BOX_SPREAD = 0.10


def _profiles_json(rel):
    try:
        with open(os.path.join(ROOT, rel)) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


def traffic_from_profiles(kernel_key):
    """HBM bytes per launch from the committed rocprofv3 PMC summary, if
    present. Not measured in this run: copied from TRAFFIC_FILE."""
    return _profiles_json(TRAFFIC_FILE).get(kernel_key)


def profile_from_profiles(kernel_key, frac):
    """The committed rocprofv3 kernel-trace figures of the headline kernel
    (PROFILE_FILE: median and mean dispatch time and the fraction they give,
    the summary file, and the bench line printed in that same profiled run),
    with how far this run's fraction lies from the profile's."""
    rec = _profiles_json(PROFILE_FILE).get(kernel_key)
    if not rec:
        return None
    out = dict(rec)
    out["this_run_vs_profile"] = round(frac / rec["frac"] - 1.0, 4)
    out["within_box_spread"] = abs(frac / rec["frac"] - 1.0) <= BOX_SPREAD
    return out


def cpu_threads(torch):
    """Every host core for the CPU baseline (torch.set_num_threads(os.cpu_count()));
    returns the count used."""
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    return threads


def cpu_timed(torch, fn, reps=2):
    """Host wall seconds per call of the reference CPU path: one warm-up, then
    the mean of `reps` calls."""
    fn()
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    return (time.perf_counter() - t0) / reps


def cpu_entry(torch, seconds, flop, sample, threads):
    return {"ms": round(seconds * 1e3, 3), "GFLOP/s": round(flop / seconds / 1e9, 2), "cores": threads,
            "kind": "port", "sample": sample}


def cpu_mp2_baseline(torch, seconds=12.0):
    """Reference CPU loop (oracle/cpu_ref.py, trntensor/quantum.py:87-100) on
    config-4 fp64 inputs, over as many ordered (i, j) pairs as fit in about
    `seconds`; scaled to the full 4096-pair job and reported in the GPU's unit
    (algorithmic GFLOP/s over the i<=j work)."""
    from oracle import cpu_ref

    threads = cpu_threads(torch)
    B, eo, ev = mp2_inputs(torch, torch.float64)
    nocc = B.shape[0]
    pairs = [(i, j) for i in range(nocc) for j in range(nocc)]
    cpu_ref.mp2_energy_pairs(B, eo, ev, pairs[:4])  # warm-up
    done, t0 = 0, time.perf_counter()
    while done < len(pairs) and time.perf_counter() - t0 < seconds:
        cpu_ref.mp2_energy_pairs(B, eo, ev, pairs[done : done + 64])
        done += 64
    dt = time.perf_counter() - t0
    full = dt * len(pairs) / done
    alg = 2080 * 2 * 320**2 * 1200
    return {
        "value": round(alg / full / 1e9, 2),
        "unit": "GFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{done} of {len(pairs)} ordered (i,j) pairs of the reference loop in {dt:.1f} s, "
        f"scaled to the full loop ({full:.1f} s); torch {torch.__version__} CPU",
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(
            f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no multi-GPU path. "
            "Run with --gpus 1.",
            file=sys.stderr,
        )
        sys.exit(2)
    import torch

    import trntensor_amd as tt
    from trntensor_amd.hip import dispatch

    if not dispatch.HAS_HIP:
        raise SystemExit(f"HIP path unavailable: {dispatch._UNAVAILABLE_REASON}")
    dev = torch.device("cuda", 0)
    if args.calibrate_copy:
        x = torch.ones(1 << 27, dtype=torch.float64, device=dev)
        y = torch.empty_like(x)
        for _ in range(5):
            y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes_read": x.numel() * 8, "bytes_written": y.numel() * 8, "launches": 5}))
        return
    if args.skip_headline:
        extra = {}
        want = set(filter(None, args.only.split(","))) or {"c1", "c2", "c3", "c4f32", "c4naux", "c5", "f1", "a5"}
        if "c3" in want:
            extra["c3_ao_to_mo_half_fp64"] = bench_c3(torch, tt, dev, args)
        if "c4f32" in want:
            extra["c4_mp2_fp32"] = bench_c4_f32(torch, tt, dev, args)
        if "c4naux" in want:
            extra["c4_mp2_naux_sweep"] = bench_c4_naux(torch, tt, dev, args)
        if "c2" in want:
            extra["c2"] = bench_c2(torch, tt, dev, args)
        if "c1" in want:
            extra["c1_einsum_loop_fp32"] = bench_c1(torch, tt, dev, args)
        if "c5" in want:
            extra["c5_greedy_path_fp64"] = bench_c5(torch, tt, dev, args)
        if "f1" in want:
            extra["f1_ao_to_mo_full_then_mp2_fp64"] = bench_f1(torch, tt, dev, args)
        if "a5" in want:
            extra["a5_strided_patterns"] = bench_a5(torch, tt, dev, args)
        print(json.dumps({"configs": extra}))
        return

    # ---------------- headline: config 4, fp64 --------------------------------
    B, eo, ev = (x.to(dev) for x in mp2_inputs(torch, torch.float64))
    flop = 2080 * 2 * 320**2 * 1200
    print("bench: mp2_energy fp64 64x320x1200", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    wall, ev_ms, ev_med = timed(torch, lambda: tt.mp2_energy(B, eo, ev), args.steps, args.warmup)
    value = flop / (wall * 1e-3) / 1e9
    achieved = flop / (ev_ms * 1e-3)
    kernel_key = "mp2_energy_kernel<double>"
    line = {
        "metric": "DF-MP2 energy GFLOP/s + % fp64 MFMA peak; AO->MO GB/s, 1 MI355X",
        "value": round(value, 1),
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64",
        "data": "synthetic (seeded torch.Generator, BASELINE config-4 distributions)",
        "config": {
            "workload": "mp2_energy fp64 nocc=64 nvir=320 naux=1200 (BASELINE config 4), inputs resident in HBM",
            "global_batch": 1,
            "flop_per_step": flop,
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "mp2_energy_kernel<double>",
            "achieved": round(achieved / 1e12, 2),
            "peak": 78.6,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK["f64"], 4),
            "traffic": traffic_from_profiles(kernel_key),
            "traffic_source": TRAFFIC_FILE + " (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; calibrated; not this run)",
            # The byte counters see every L2 miss; the DRAM-request counter
            # (TCC_EA0_RDREQ_DRAM) reads the same 33 GB, so MALL hits are
            # included. B (197 MB) fits the 256 MB MALL: the panel re-reads of
            # the 64 x 64 work units are served there.
            "traffic_scope": "L2 misses (MALL hits + HBM); B fits the 256 MB MALL",
            "algorithmic_bytes": int(B.numel() * B.element_size() + (eo.numel() + ev.numel()) * 8),
            "event_ms_per_launch": round(ev_ms, 4),
            "event_ms_median": round(ev_med, 4),
            "frac_at_median": round(flop / (ev_med * 1e-3) / PEAK["f64"], 4),
            "box_spread": BOX_SPREAD,
            "profile": profile_from_profiles(kernel_key, achieved / PEAK["f64"]),
        },
    }
    del B, eo, ev
    print("bench: measured peaks (MFMA probe, device copy)", file=sys.stderr, flush=True)
    peaks = measured_peaks(torch, dev)
    line["measured_peaks"] = peaks
    line["roofline"]["frac_measured_peak"] = round(achieved / 1e12 / peaks["mfma_f64_TFLOPs"], 4)

    extra = {}
    want = set(filter(None, args.only.split(","))) or {"c1", "c2", "c3", "c4f32", "c4naux", "c5", "f1", "a5"}
    if not args.no_extra:
        if "c3" in want:
            extra["c3_ao_to_mo_half_fp64"] = bench_c3(torch, tt, dev, args)
            line["ao_to_mo_GBps"] = extra["c3_ao_to_mo_half_fp64"]["GB/s"]
        if "c4f32" in want:
            extra["c4_mp2_fp32"] = bench_c4_f32(torch, tt, dev, args)
        if "c4naux" in want:
            extra["c4_mp2_naux_sweep"] = bench_c4_naux(torch, tt, dev, args)
        if "c2" in want:
            extra["c2"] = bench_c2(torch, tt, dev, args)
        if "c1" in want:
            extra["c1_einsum_loop_fp32"] = bench_c1(torch, tt, dev, args)
        if "c5" in want:
            extra["c5_greedy_path_fp64"] = bench_c5(torch, tt, dev, args)
        if "f1" in want:
            extra["f1_ao_to_mo_full_then_mp2_fp64"] = bench_f1(torch, tt, dev, args)
        if "a5" in want:
            extra["a5_strided_patterns"] = bench_a5(torch, tt, dev, args)
        line["measured_peaks"]["fractions_above_1"] = add_measured_fractions(extra, peaks)
        line["configs"] = extra

    if not args.no_cpu:
        print("bench: cpu baseline (reference loop sample)", file=sys.stderr, flush=True)
        line["cpu_baseline"] = cpu_mp2_baseline(torch)
        line["cpu_baseline"]["host"] = host_info(torch)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


def bench_c3(torch, tt, dev, args):
    print("bench: c3 ao->mo half", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(0)
    C = torch.linalg.qr(torch.randn(512, 64, generator=g, dtype=torch.float64))[0].contiguous().to(dev)
    eri = torch.randn(512, 512, 1536, generator=g, dtype=torch.float64).to(dev)
    eri = ((eri + eri.permute(1, 0, 2)) * (0.05 / 2**0.5)).contiguous()
    wall, ev_ms = timed_steady(torch, lambda: tt.einsum("mi,mnP->inP", C, eri), max(5, args.steps))
    byt = (512 * 512 * 1536 + 64 * 512 * 1536 + 512 * 64) * 8
    flop = 2 * 64 * 512 * 512 * 1536
    t = ev_ms * 1e-3
    t_floor = max(flop / PEAK["f64"], byt / PEAK["hbm"])
    cpu = None
    if not args.no_cpu:
        from oracle import cpu_ref

        threads = cpu_threads(torch)
        Cc, ec = C.cpu(), eri.cpu()
        del eri
        sec = cpu_timed(torch, lambda: cpu_ref.einsum("mi,mnP->inP", Cc, ec))
        cpu = cpu_entry(torch, sec, flop, "full config 3 through the reference's 'torch' strategy (torch.einsum)", threads)
        del Cc, ec
    return {
        "cpu": cpu,
        "ms": round(ev_ms, 4),
        "wall_ms": round(wall, 4),
        "GB/s": round(byt / t / 1e9, 1),
        "TFLOP/s": round(flop / t / 1e12, 2),
        "frac_hbm": round(byt / t / PEAK["hbm"], 4),
        "frac_mfma": round(flop / t / PEAK["f64"], 4),
        "frac_binding_roofline": round(t_floor / t, 4),
        "bound": "mfma (AI 14.2 flop/B > fp64 ridge 9.8)",
        "kernel": "gemm_directb_stream_kernel (A through LDS, B streamed into registers)",
    }


def bench_a5(torch, tt, dev, args):
    """'torch'-strategy contractions without a GEMM shape (tt_strided_contract):
    HBM-bound permutations and reductions on 1 GiB operands. Bytes = operand
    read once + output written once; bound = HBM."""
    print("bench: a5 strided patterns", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(0)
    X = torch.randn(512, 512, 512, generator=g, dtype=torch.float64)
    T = torch.randn(16384, 16384, generator=g, dtype=torch.float32)
    Xd, Td = X.to(dev), T.to(dev)
    cases = [
        ("ijk->kji", Xd, X, 2 * X.numel() * 8),
        ("ijk->ikj", Xd, X, 2 * X.numel() * 8),
        ("ijk->k", Xd, X, X.numel() * 8),
        ("ijk->i", Xd, X, X.numel() * 8),
        ("ij->ji", Td, T, 2 * T.numel() * 4),
    ]
    out = {}
    for sub, d, h, byt in cases:
        _, ms = timed_steady(torch, lambda: tt.einsum(sub, d), max(5, args.steps))
        r = {"ms": round(ms, 4), "GB/s": round(byt / (ms * 1e-3) / 1e9, 1),
             "frac_hbm": round(byt / (ms * 1e-3) / PEAK["hbm"], 4)}
        if not args.no_cpu:
            from oracle import cpu_ref

            threads = cpu_threads(torch)
            # torch.einsum returns a permuted view for a pure permutation; the
            # baseline materialises it (.contiguous()) like the GPU result.
            sec = cpu_timed(torch, lambda: cpu_ref.einsum(sub, h).contiguous(), reps=1)
            r["cpu"] = {"ms": round(sec * 1e3, 2), "GB/s": round(byt / sec / 1e9, 2), "cores": threads, "kind": "port",
                        "sample": "full operand through the reference's 'torch' strategy (torch.einsum), "
                                  "materialised with .contiguous()"}
        out[f"{sub} {str(h.dtype).replace('torch.', '')}"] = r
    return out


def bench_f1(torch, tt, dev, args):
    """Full AO->MO transform at config-3 sizes with nvir = 320 (B[64, 320, 1536]),
    then the fused MP2 energy on the device-resident B: the DF-MP2 pipeline
    with nothing leaving HBM."""
    print("bench: f1 ao->mo full + mp2", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(0)
    C = torch.linalg.qr(torch.randn(512, 384, generator=g, dtype=torch.float64))[0]
    C_occ, C_vir = C[:, :64].contiguous().to(dev), C[:, 64:].contiguous().to(dev)
    eri = torch.randn(512, 512, 1536, generator=g, dtype=torch.float64).to(dev)
    eri = ((eri + eri.permute(1, 0, 2)) * (0.05 / 2**0.5)).contiguous()
    eo = torch.sort(-20 + 19.7 * torch.rand(64, generator=g, dtype=torch.float64))[0].to(dev)
    ev = torch.sort(0.1 + 4.9 * torch.rand(320, generator=g, dtype=torch.float64))[0].to(dev)
    flop_t = 2 * 64 * 512 * 512 * 1536 + 2 * 64 * 320 * 1536 * 512
    flop_e = 2080 * 2 * 320**2 * 1536
    _, ms_t = timed_steady(torch, lambda: tt.ao_to_mo_transform(eri, C_occ, C_vir), max(5, args.steps))
    _, ms_p = timed_steady(torch, lambda: tt.mp2_energy(tt.ao_to_mo_transform(eri, C_occ, C_vir), eo, ev), 5)
    return {
        "ao_to_mo_ms": round(ms_t, 4),
        "ao_to_mo_TFLOP/s": round(flop_t / (ms_t * 1e-3) / 1e12, 2),
        "ao_to_mo_frac_mfma": round(flop_t / (ms_t * 1e-3) / PEAK["f64"], 4),
        "pipeline_ms": round(ms_p, 3),
        "pipeline_TFLOP/s": round((flop_t + flop_e) / (ms_p * 1e-3) / 1e12, 2),
        "shape": "eri[512,512,1536], C_occ[512,64], C_vir[512,320] -> B[64,320,1536] -> E",
    }


def bench_c4_f32(torch, tt, dev, args):
    print("bench: c4 mp2 fp32", file=sys.stderr, flush=True)
    B, eo, ev = (x.to(dev) for x in mp2_inputs(torch, torch.float32))
    wall, ev_ms = timed_steady(torch, lambda: tt.mp2_energy(B, eo, ev), args.steps)
    flop = 2080 * 2 * 320**2 * 1200
    cpu = None
    if not args.no_cpu:
        from oracle import cpu_ref

        threads = cpu_threads(torch)
        Bc, eoc, evc = B.cpu(), eo.cpu(), ev.cpu()
        pairs = [(i, j) for i in range(64) for j in range(64)]
        sec = cpu_timed(torch, lambda: cpu_ref.mp2_energy_pairs(Bc, eoc, evc, pairs[:256]), reps=1) * 16
        cpu = cpu_entry(torch, sec, flop, "256 of 4096 ordered (i,j) pairs of the reference loop, scaled x16", threads)
    return {
        "cpu": cpu,
        "ms": round(ev_ms, 4),
        "GFLOP/s": round(flop / (wall * 1e-3) / 1e9, 1),
        "frac_mfma_f32": round(flop / (ev_ms * 1e-3) / PEAK["f32"], 4),
    }


def bench_c4_naux(torch, tt, dev, args):
    """Config 4 with auxiliary sizes that are not multiples of 16 (real
    auxiliary basis sizes are arbitrary). Each call (timed whole) first copies
    B into the workspace with rows padded to a multiple of 16 elements, so
    every stage of the kernel reads aligned cache lines. Also nvir 300 (not a
    multiple of the 64-row block) and a problem past the MALL."""
    out = {}
    for dt, key, peak in ((torch.float64, "f64", PEAK["f64"]), (torch.float32, "f32", PEAK["f32"])):
        for naux in (1200, 1190, 1199, 1201):
            print(f"bench: c4 naux {naux} {key}", file=sys.stderr, flush=True)
            B, eo, ev = (x.to(dev) for x in mp2_inputs(torch, dt, naux=naux))
            _, ms = timed_steady(torch, lambda: tt.mp2_energy(B, eo, ev), max(5, args.steps))
            flop = 2080 * 2 * 320**2 * naux
            out[f"{key}_naux{naux}"] = {"ms": round(ms, 4), "TFLOP/s": round(flop / (ms * 1e-3) / 1e12, 2),
                                        "frac_mfma": round(flop / (ms * 1e-3) / peak, 4)}
            del B, eo, ev
        # nvir not a multiple of the 64-row block (a 44-row last block): the
        # fraction counts algorithmic FLOP only, so the padded rows' work is
        # overhead here.
        print(f"bench: c4 nvir 300 {key}", file=sys.stderr, flush=True)
        B, eo, ev = (x.to(dev) for x in mp2_inputs(torch, dt, nvir=300))
        _, ms = timed_steady(torch, lambda: tt.mp2_energy(B, eo, ev), max(5, args.steps))
        flop = 2080 * 2 * 300**2 * 1200
        out[f"{key}_nvir300"] = {"ms": round(ms, 4), "TFLOP/s": round(flop / (ms * 1e-3) / 1e12, 2),
                                 "frac_mfma": round(flop / (ms * 1e-3) / peak, 4)}
        del B, eo, ev
    # A production-sized problem whose B (1.57 GB) does not fit the 256 MB
    # MALL, so the panel re-reads that miss L2 go to HBM (inputs drawn on the
    # device; same distributions as config 4).
    print("bench: mp2 128x640x2400 fp64", file=sys.stderr, flush=True)
    g = torch.Generator(device=dev).manual_seed(0)
    B = torch.randn(128, 640, 2400, generator=g, device=dev, dtype=torch.float64) * 0.05
    eo = torch.sort(-20 + 19.7 * torch.rand(128, generator=g, device=dev, dtype=torch.float64))[0]
    ev = torch.sort(0.1 + 4.9 * torch.rand(640, generator=g, device=dev, dtype=torch.float64))[0]
    _, ms = timed_steady(torch, lambda: tt.mp2_energy(B, eo, ev), 3)
    flop = (128 * 129 // 2) * 2 * 640**2 * 2400
    out["f64_nocc128_nvir640_naux2400"] = {"ms": round(ms, 2), "TFLOP/s": round(flop / (ms * 1e-3) / 1e12, 2),
                                           "frac_mfma": round(flop / (ms * 1e-3) / PEAK["f64"], 4),
                                           "B_GB": round(B.numel() * 8 / 1e9, 2)}
    del B, eo, ev
    # One GPU's share of an 8-GPU run at config 4 (fp64): each shard is a
    # contiguous eighth of the 31,200 work units (tt_mp2_energy_shard).
    print("bench: c4 shards of 8", file=sys.stderr, flush=True)
    B, eo, ev = (x.to(dev) for x in mp2_inputs(torch, torch.float64))
    shard_ms = []
    for r in range(8):
        _, ms = timed_steady(torch, lambda: tt.mp2_energy_shard(B, eo, ev, r, 8), max(5, args.steps))
        shard_ms.append(ms)
    _, whole_ms = timed_steady(torch, lambda: tt.mp2_energy(B, eo, ev), max(5, args.steps))
    out["f64_shard_of_8"] = {"max_ms": round(max(shard_ms), 4), "min_ms": round(min(shard_ms), 4),
                             "sum_ms": round(sum(shard_ms), 4), "whole_ms": round(whole_ms, 4),
                             "balance": round(min(shard_ms) / max(shard_ms), 4)}
    return out


def bench_c2(torch, tt, dev, args):
    out = {}
    g = torch.Generator().manual_seed(0)
    for name, shape, sub, flop in (
        ("gemm4096", (4096, 4096), "ij,jk->ik", 2 * 4096**3),
        ("bmm64x512", (64, 512, 512), "bij,bjk->bik", 64 * 2 * 512**3),
    ):
        for dt, key in ((torch.float64, "f64"), (torch.float32, "f32"), (torch.bfloat16, "bf16")):
            print(f"bench: c2 {name} {key}", file=sys.stderr, flush=True)
            hostA, hostB, hostC = (torch.randn(*shape, generator=g, dtype=torch.float64).to(dt) for _ in range(3))
            A, B, C = (x.to(dev) for x in (hostA, hostB, hostC))
            wall, ev_ms = timed_steady(torch, lambda: tt.einsum(sub, A, B, alpha=1.5, beta=0.5, out=C), max(5, args.steps))
            # Library comparator on the same operands: hipBLASLt/rocBLAS through torch.
            lib_fn = torch.addmm if A.dim() == 2 else torch.baddbmm
            _, lib_ms = timed_steady(torch, lambda: lib_fn(C, A, B, beta=0.5, alpha=1.5), max(5, args.steps))
            out[f"{name}_{key}"] = {
                "ms": round(ev_ms, 4),
                "TFLOP/s": round(flop / (ev_ms * 1e-3) / 1e12, 2),
                "frac_mfma": round(flop / (ev_ms * 1e-3) / PEAK[key], 4),
                "torch_rocm_lib_TFLOP/s": round(flop / (lib_ms * 1e-3) / 1e12, 2),
            }
            if key == "bf16":
                # The reference has no bf16 config; this line times the 16-bit
                # MFMA GEMM (einsum on bf16 operands), without a CPU leg.
                del A, B, C, hostA, hostB, hostC
                continue
            if not args.no_cpu:
                from oracle import cpu_ref

                threads = cpu_threads(torch)
                sec = cpu_timed(torch, lambda: cpu_ref.einsum(sub, hostA, hostB, alpha=1.5, beta=0.5, out=hostC))
                out[f"{name}_{key}"]["cpu"] = cpu_entry(
                    torch, sec, flop, "full config through the reference's matmul/bmm executor plus the alpha/beta passes", threads)
            del A, B, C, hostA, hostB, hostC
    # precision="dd": double-double on the vector ALUs. Dot2 costs 10
    # double-precision VALU operations per multiply-add; the ceiling is the
    # fp64 vector rate, 78.6 TFLOP/s = 39.3e12 operations/s.
    print("bench: c2 gemm4096 dd", file=sys.stderr, flush=True)
    A, B = (torch.randn(4096, 4096, generator=g, dtype=torch.float64).to(dev) for _ in range(2))
    wall, ev_ms = timed_steady(torch, lambda: tt.einsum("ij,jk->ik", A, B, precision="dd"), 3)
    mac = 4096**3
    out["gemm4096_dd"] = {
        "ms": round(ev_ms, 3),
        "TMAC/s": round(mac / (ev_ms * 1e-3) / 1e12, 3),
        "frac_valu": round(10 * mac / (ev_ms * 1e-3) / 39.3e12, 4),
    }
    return out


def bench_c1(torch, tt, dev, args):
    """examples/df_mp2_einsum.py loop at config 1 with trntensor_amd.einsum per pair
    (CPU operands, as in the config) and the fused call on the same CPU tensors."""
    print("bench: c1 einsum loop", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(0)
    B = torch.randn(8, 32, 96, generator=g) * 0.1
    eo = torch.sort(-20 + 19.7 * torch.rand(8, generator=g))[0]
    ev = torch.sort(0.1 + 4.9 * torch.rand(32, generator=g))[0]

    def loop():
        e = 0.0
        for i in range(8):
            for j in range(8):
                T = tt.einsum("ap,bp->ab", B[i], B[j])
                d = eo[i] + eo[j] - ev.unsqueeze(1) - ev.unsqueeze(0)
                e += (T * (2 * T - T.T) / d).sum().item()
        return e

    def per_call(fn, reps, warm_s=0.3):
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < warm_s:
            fn()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        return (time.perf_counter() - t0) / reps

    t_loop = per_call(loop, 10)
    t_fused = per_call(lambda: float(tt.mp2_energy(B, eo, ev)), 50)
    res = {"einsum_loop_ms": round(t_loop * 1e3, 3), "fused_cpu_operands_ms": round(t_fused * 1e3, 3)}
    # The loop's 64 contractions on device-resident operands: eager calls, and
    # the same calls recorded once in a HIP graph and replayed (launch-bound
    # loops are what graphs are for; the library allocates nothing and issues
    # no memsets, so its launches record as plain kernel nodes).
    Bd = B.to(dev)

    def dev_loop():
        return [tt.einsum("ap,bp->ab", Bd[i], Bd[j]) for i in range(8) for j in range(8)]

    def synced(fn):
        def run():
            fn()
            torch.cuda.synchronize()
        return run

    t_dev = per_call(synced(dev_loop), 20)
    # Host cost per call alone: the 64 launches enqueued back to back (the
    # queue holds them all), timed before the synchronisation.
    host = []
    for _ in range(20):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        dev_loop()
        host.append((time.perf_counter() - t0) / 64)
    torch.cuda.synchronize()
    res["device_einsum_host_us_per_call"] = round(statistics.median(host) * 1e6, 2)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        dev_loop()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        dev_loop()
    t_graph = per_call(synced(graph.replay), 50)
    res["device_einsum_loop_ms"] = round(t_dev * 1e3, 3)
    res["device_einsum_loop_graph_replay_ms"] = round(t_graph * 1e3, 3)
    # The reference's residency test (tests/test_nki_kernels.py): five 2048^2
    # fp32 products on host operands against the same on device-resident ones.
    Ah, Bh = torch.randn(2048, 2048, generator=g), torch.randn(2048, 2048, generator=g)
    Ad, Bdd = Ah.to(dev), Bh.to(dev)
    t_cold = per_call(lambda: tt.einsum("ij,jk->ik", Ah, Bh), 5, 0.1)
    t_hot = per_call(synced(lambda: tt.einsum("ij,jk->ik", Ad, Bdd)), 5, 0.1)
    res["residency_speedup_2048"] = round(t_cold / t_hot, 2)
    if not args.no_cpu:
        from oracle import cpu_ref

        threads = cpu_threads(torch)
        sec = per_call(lambda: cpu_ref.df_mp2_einsum_loop(B, eo, ev), 10)
        res["cpu"] = {"einsum_loop_ms": round(sec * 1e3, 3), "cores": threads, "kind": "port",
                      "sample": "the reference example loop (64 einsum calls) on the same CPU tensors"}
    return res


def bench_c5(torch, tt, dev, args):
    print("bench: c5 greedy path", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(0)
    A = (torch.randn(128, 400, generator=g, dtype=torch.float64) * 0.1).to(dev)
    B = (torch.randn(128, 400, generator=g, dtype=torch.float64) * 0.1).to(dev)
    W = (torch.randn(400, 400, 800, generator=g, dtype=torch.float64) * 0.01).to(dev)
    V = (torch.randn(128, 128, 800, generator=g, dtype=torch.float64) * 0.1).to(dev)
    wall, ev_ms = timed_steady(torch, lambda: tt.einsum("ia,jb,abP,ijP->", A, B, W, V), 3)
    flop = 2.62144e9 + 2 * 2.097152e12 + 2 * 2.62144e9
    res = {"ms": round(ev_ms, 3), "TFLOP/s": round(flop / (ev_ms * 1e-3) / 1e12, 2),
           "frac_mfma": round(flop / (ev_ms * 1e-3) / PEAK["f64"], 4), "path": "reference greedy [(0,1),(0,1),(0,1)]"}
    # opt-in fewest-multiply-add order: 2*(1.6384e10 + 5.24288e9 + 51200) flop
    wall, ev_ms = timed_steady(torch, lambda: tt.einsum("ia,jb,abP,ijP->", A, B, W, V, optimize="optimal"), 10)
    flop = 2 * (1.6384e10 + 5.24288e9 + 51200)
    res["optimize_optimal"] = {"ms": round(ev_ms, 3), "TFLOP/s": round(flop / (ev_ms * 1e-3) / 1e12, 2),
                               "frac_mfma": round(flop / (ev_ms * 1e-3) / PEAK["f64"], 4),
                               "path": "[(1,2),(1,2),(0,1)]", "speedup": round(res["ms"] / ev_ms, 1)}
    if not args.no_cpu:
        from oracle import cpu_ref

        threads = cpu_threads(torch)
        # Sample: a restricted to 40 of 400. The greedy path keeps its order
        # ([(0,1),(0,1),(0,1)]: the first pair stays cheapest) and every
        # step's work is linear in a, so the time scales by 10.
        Ac, Bc, Wc, Vc = A[:, :40].cpu(), B.cpu(), W[:40].cpu(), V.cpu()
        assert cpu_ref.plan_contraction("ia,jb,abP,ijP->", Ac, Bc, Wc, Vc).contraction_path == [(0, 1), (0, 1), (0, 1)]
        sec = cpu_timed(torch, lambda: cpu_ref.einsum("ia,jb,abP,ijP->", Ac, Bc, Wc, Vc), reps=1) * 10
        res["cpu"] = cpu_entry(torch, sec, 2.62144e9 + 2 * 2.097152e12 + 2 * 2.62144e9,
                               "reference greedy path with a restricted to 40 of 400 (same path, work linear in a), x10",
                               threads)
    return res


if __name__ == "__main__":
    main()
