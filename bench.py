"""Benchmark of the north-star path: fused masked sample + log-probability at
[S=1, B=256, T=1, V=128256] bf16 with a u8 grammar mask and temperature 0.7 (benchmark configuration 4).

One step = one launch of nt_hip_rl_sample over the 256 rows, inputs resident in HBM (the
per-step uniforms are uploaded before the timed region) and cycled over copies totalling 1 GiB,
so that no launch finds its input in the 256 MB Infinity Cache. The timed region is K
back-to-back launches bracketed by a stream synchronisation and HIP events recorded on the
library's own stream; the same launches re-reading one input are reported as `warm_cache`. Prints one JSON line (the driver's contract) with a `roofline` object (algorithmic
bytes per launch / average launch time against the 8 TB/s HBM peak) and a `cpu_baseline`
object (the reference's Cpu(Reference) op sequence, restated in oracle/, timed on this host).

`--workload c4s|c4f|c4g|c2|c3|c3b|c5|matmul|readout` measures the other configurations the same way, one
JSON line each:
  c4s C4 with one u8 grammar mask [1,V] shared by every row (mask_ld 0);
  c4f C4's rows under the reference's own mask form, the same grammar mask as an f32 additive
      0 / -inf mask [256,V] (the streaming sampler);
  c4g C4's rows through the reference's own Gumbel-max sample_categorical (one u64 per logit,
      generated on the device at the stream's position; nt_hip_rl_sample_gumbel);
  c2  decode step, f32 [1,64,1,32000], no mask, tau 0.8: the fused sample + logp;
  c3  PPO scoring, bf16 policy + reference [8,16,512,50304]: logp, reference logp, exact KL,
      entropy (nt_hip_rl_score) and the k3 per-token KL (nt_hip_rl_kl_estimate);
  c3b the c3 scoring forward plus its fused backward (nt_hip_rl_score_backward): the gradient
      of g_logp logp + g_kl KL + g_H H with respect to the logits, in bf16;
  c5  rollout scoring, f32 [4,32,1024,151936] + u8 mask: logp and entropy (nt_hip_rl_score),
      the per-sequence mean log-probability (nt_hip_rl_reduce_tokens) and group-relative
      advantages over groups of 8 along B (nt_hip_rl_group_advantages, f64 on the device);
  matmul  the general ops' f32 matmul (CpuRef's arithmetic) at the reference's throughput
      shapes and 4096^3;
  readout  C4's decode step from the hidden states: h[256,4096] . W (V 128256) fused with the
      sample + logp (nt_hip_rl_readout_sample), and with the scoring of the drawn tokens
      (nt_hip_rl_readout_score), each beside hipBLASLt's GEMM and the unfused kernel.
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "noetic-tensor_amd"))

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0  # MI355X published HBM3E bandwidth


def hip_events():
    """hipEvent* from the HIP runtime the library itself links."""
    hip = C.CDLL("libamdhip64.so")
    hip.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
    hip.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
    hip.hipEventSynchronize.argtypes = [C.c_void_p]
    hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
    hip.hipEventDestroy.argtypes = [C.c_void_p]
    return hip


def cpu_model():
    """The host CPU's model name (Linux /proc/cpuinfo), for the baseline's record."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def copy_peak(nr, nbytes=1 << 29, reps=10):
    """A measured streaming-copy rate on this device: device-to-device hipMemcpyAsync of nbytes on
    the library's stream, read + write bytes over the HIP-event time (GB/s)."""
    hip = hip_events()
    hip.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
    src, dst = nr.Buffer(nbytes), nr.Buffer(nbytes)
    stream = C.c_void_p()
    nr._check(nr.lib().nt_hip_stream(C.byref(stream)), "stream")
    d2d = 3  # hipMemcpyDeviceToDevice
    for _ in range(2):
        hip.hipMemcpyAsync(C.c_void_p(dst.ptr), C.c_void_p(src.ptr), nbytes, d2d, stream)
    nr.sync()
    e0, e1 = C.c_void_p(), C.c_void_p()
    hip.hipEventCreate(C.byref(e0))
    hip.hipEventCreate(C.byref(e1))
    hip.hipEventRecord(e0, stream)
    for _ in range(reps):
        hip.hipMemcpyAsync(C.c_void_p(dst.ptr), C.c_void_p(src.ptr), nbytes, d2d, stream)
    hip.hipEventRecord(e1, stream)
    hip.hipEventSynchronize(e1)
    ms = C.c_float()
    hip.hipEventElapsedTime(C.byref(ms), e0, e1)
    hip.hipEventDestroy(e0)
    hip.hipEventDestroy(e1)
    return 2 * nbytes * reps / (ms.value * 1e-3) / 1e9


def clock_warmup(nr, step, seconds):
    """Run `step(i)` untimed for about `seconds` of wall time (synchronising every 64 calls), so
    that the timed windows that follow see the device's steady clocks: MI355X raises its shader
    clock over the first tenths of a second of sustained work (a kernel measured 343 us at the
    start of a run and 260-275 us after one second of it)."""
    t0 = time.perf_counter()
    i = 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(64):
            step(i)
            i += 1
        nr.sync()
    return time.perf_counter() - t0


def timed(nr, steps, warmup, step):
    """Average milliseconds of `step(i)` over `steps` calls after `warmup` untimed ones, from HIP
    events on the library's stream (where every kernel runs), plus the wall seconds."""
    for i in range(warmup):
        step(i)
    nr.sync()
    hip = hip_events()
    stream = C.c_void_p()
    nr._check(nr.lib().nt_hip_stream(C.byref(stream)), "stream")
    e0, e1 = C.c_void_p(), C.c_void_p()
    hip.hipEventCreate(C.byref(e0))
    hip.hipEventCreate(C.byref(e1))
    nr.sync()
    t0 = time.perf_counter()
    hip.hipEventRecord(e0, stream)
    for i in range(warmup, warmup + steps):
        step(i)
    hip.hipEventRecord(e1, stream)
    hip.hipEventSynchronize(e1)
    nr.sync()
    wall = time.perf_counter() - t0
    ms = C.c_float()
    hip.hipEventElapsedTime(C.byref(ms), e0, e1)
    hip.hipEventDestroy(e0)
    hip.hipEventDestroy(e1)
    return ms.value / steps, wall


def practical_floor(nr, bytes_launch, traffic, ms, blocks):
    """The practical floor of one launch on this box, measured in this run with the library's own
    kernels (include/noetic_measure.h): the device's streaming-read rate over 2 GiB (beyond the
    Infinity Cache) and the period of back-to-back launches of a kernel that does nothing, with
    the sampler's grid (one 1024-thread workgroup per row). floor = period + bytes / read rate,
    for the algorithmic bytes and for the HBM bytes the counters measured (`traffic`)."""
    L = nr.lib()
    gbs, us = C.c_double(), C.c_double()
    nr._check(L.nt_measure_read(C.c_size_t(2 << 30), 10, C.byref(gbs)), "measure read")
    nr._check(L.nt_measure_launch_period(blocks, 1024, 2000, C.byref(us)), "measure launch period")
    out = {"read_gbs": gbs.value, "launch_period_us": us.value,
           "floor_us": us.value + bytes_launch / (gbs.value * 1e3),
           "what": "floor = launch period + algorithmic bytes / measured read rate; frac_of_floor = floor / launch time"}
    out["frac_of_floor"] = out["floor_us"] / (ms * 1e3)
    if traffic:
        out["floor_us_on_traffic"] = us.value + traffic / (gbs.value * 1e3)
    return out


def valu_roofline(nr, ms, counters_file):
    """A VALU-bound kernel's roofline: its VALU instructions per launch (SQ_INSTS_VALU, read from
    the committed rocprofv3 summary `counters_file`) over the launch time, against the issue
    capacity of the chip's SIMDs: 256 CUs x 4 SIMDs, one 64-lane instruction every 4 cycles each
    (16 lanes wide), at the shader clock measured in this run under a load of dependent fused
    multiply-adds on every SIMD (include/noetic_measure.h). `achieved` and `peak` are in G
    wave-instructions/s."""
    mhz = C.c_double()
    nr._check(nr.lib().nt_measure_shader_clock(1000, C.byref(mhz)), "measure shader clock")
    peak = 256 * 4 * mhz.value * 1e6 / 4 / 1e9
    path = os.path.join(ROOT, "profiles", counters_file)
    n = achieved = None
    if os.path.exists(path):  # (absent while the counters themselves are being collected)
        with open(path) as f:
            n = json.load(f)["sq_insts_valu_per_dispatch"]
        achieved = n / (ms * 1e-3) / 1e9
    return {"bound": "valu", "achieved": achieved, "peak": peak, "unit": "G wave-instructions/s",
            "frac": None if n is None else achieved / peak, "traffic": None, "valu_instructions_per_launch": n,
            "shader_clock_mhz": mhz.value,
            "what": "VALU wave-instructions per launch (SQ_INSTS_VALU) / launch time, against 256 CUs x 4 SIMDs "
                    "x one wave-instruction per 4 cycles at the measured shader clock"}


def roofline(bytes_launch, ms, traffic_file=None):
    gbs = bytes_launch / (ms * 1e-3) / 1e9
    r = {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS,
         "traffic": None, "algorithmic_bytes_per_launch": bytes_launch}
    if traffic_file:
        tr = os.path.join(ROOT, "profiles", traffic_file)
        if os.path.exists(tr):
            with open(tr) as f:
                r["traffic"] = json.load(f).get("hbm_bytes_per_launch")
    return r


def line(metric, value, steps, warmup, ms, dtype, config, roof, **extra):
    out = {"metric": metric, "value": value, "unit": "rows/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
           "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": dtype,
           "data": "synthetic", "config": config, "roofline": roof}
    out.update(extra)
    return out


def cpu_threads():
    """The Cpu(Fast) worker count: NOETIC_THREADS, else every host core (src/tensor/backend.rs:59-61)."""
    try:
        n = int(os.environ.get("NOETIC_THREADS", ""))
    except ValueError:
        n = 0
    return max(1, n or (os.cpu_count() or 1))


def cpu_baseline(w, rows_sample, seed, min_seconds=10.0, gpu=None):
    """The reference's CPU path on a bounded sample of the same rows (restated in oracle/oracle.c):
    tempered_logits, the max_dim check, one Gumbel draw per logit from the ChaCha stream, argmax,
    then token_log_probs (log_softmax and gather), in f32, on Cpu(Reference) (one thread) and on
    Cpu(Fast) (its thresholds and threading, NOETIC_THREADS workers). Also the build's own unfused
    inverse-CDF port on every core. `gpu` = (ids, logp, uniforms) of one device launch over the
    same rows: its parity against the oracle is checked here, outside any timed region."""
    import workloads as W
    from oracle import oracle as O
    V = w["V"]
    x = W.download_rows(w["logits"], range(rows_sample), V)
    x = W.bf16_to_f32(x) if w["logits"].dtype == "bf16" else x
    mrows = [0] * rows_sample if w.get("mask_shared") else range(rows_sample)
    keep = W.download_rows(w["mask"], mrows, V) if w["mask"] is not None else None
    rng = O.Rng(seed, f"{w['name']}/gumbel")
    reps, t_ref = 0, 0.0
    while reps < 1 or (t_ref < min_seconds and reps < 1000):
        t0 = time.perf_counter()
        O.cpuref_sample_logp(x, w["temperature"], keep, rng)
        t_ref += time.perf_counter() - t0
        reps += 1
    threads = cpu_threads()
    rng_f = O.Rng(seed, f"{w['name']}/gumbel")
    reps_f, t_fast = 0, 0.0
    while reps_f < 1 or (t_fast < min_seconds / 2 and reps_f < 1000):
        t0 = time.perf_counter()
        O.cpufast_sample_logp(x, w["temperature"], keep, rng_f, threads)
        t_fast += time.perf_counter() - t0
        reps_f += 1
    cores = os.cpu_count() or 1
    u = O.Rng(seed, f"{w['name']}/uniforms").uniforms(rows_sample)
    t0 = time.perf_counter()
    O.cpu_sample_logp_invcdf(x, w["temperature"], keep, u, threads=cores)
    t_inv = time.perf_counter() - t0
    out = {
        "value": reps * rows_sample / t_ref, "unit": "rows/s", "cores": 1, "kind": "port", "cpu": cpu_model(),
        "sample": f"{reps} x {rows_sample} {w['name']} rows (V={V}, values widened to f32): the reference's "
                  f"Cpu(Reference) op sequence (Gumbel-max sample_categorical, then token_log_probs), single "
                  f"thread, {t_ref:.2f} s",
        "fast": {"value": reps_f * rows_sample / t_fast, "unit": "rows/s", "cores": threads, "kind": "port",
                 "sample": f"{reps_f} x {rows_sample} rows, the same op sequence on Cpu(Fast): maps threaded from "
                           f"2^20 elements, equal-shape zips and last-axis sums from 2^22, {threads} threads "
                           f"(NOETIC_THREADS, else all cores), {t_fast:.2f} s; the Gumbel draws stay one "
                           f"sequential stream"},
        "inv_cdf_port": {"value": rows_sample / t_inv, "unit": "rows/s", "cores": cores,
                         "what": "the build's own unfused op sequence with the inverse-CDF draw (one uniform per "
                                 "row), rows split over threads; not a reference backend"},
    }
    if gpu is not None:
        out["parity"] = parity_against_oracle(O, x, keep, w["temperature"], *gpu)
    return out


def parity_against_oracle(O, x, keep, tau, ids, logp, u):
    """One device launch's ids and log-probs against the oracle's f64 inverse-CDF draw on the same
    rows and uniforms: ids must be equal except draws within 1e-6 of a CDF edge (counted), log-
    probs within the f32 tolerance (1e-5 relative, 1e-6 absolute; the bf16 inputs are exact in
    f32). The largest errors observed are reported."""
    z = O.tempered(x, tau, keep=keep)
    want, edges = O.sample_invcdf(z, u)
    boundary = edges < 1e-6
    differ = ids != want
    ref_lp = O.token_logp(z, ids)
    err = np.abs(logp.astype(np.float64) - ref_lp)
    ok = bool(np.all(boundary[differ]) and np.all(err <= 1e-6 + 1e-5 * np.abs(ref_lp)))
    return {"rows": int(len(ids)), "ids_differ": int(differ.sum()), "boundary_draws": int(boundary.sum()),
            "ids_differ_off_boundary": int((differ & ~boundary).sum()),
            "logp_max_abs_err": float(err.max()), "logp_max_rel_err": float(np.max(err / np.maximum(np.abs(ref_lp), 1e-30))),
            "logp_max_ref_tol": float(np.max(err / (1.0 + np.abs(ref_lp)))),
            "tolerance": "ids exact except |u - CDF edge| < 1e-6; logp |d| <= 1e-6 + 1e-5 |ref| (f32)",
            "within_tolerance": ok}


def cpu_baseline_scoring(w, rows_sample, min_seconds=10.0):
    """The oracle's scoring of a bounded row sample on one host core: tempered values, then
    log-softmax at the token, exact KL and entropy per row (f64 after the f32 inputs)."""
    import workloads as W
    from oracle import oracle as O
    V = w["V"]
    x = W.download_rows(w["logits"], range(rows_sample), V)
    x = W.bf16_to_f32(x) if w["logits"].dtype == "bf16" else x
    keep = W.download_rows(w["mask"], range(rows_sample), V) if w.get("mask") is not None else None
    y = None
    if w.get("ref") is not None:
        y = W.download_rows(w["ref"], range(rows_sample), V)
        y = W.bf16_to_f32(y) if w["ref"].dtype == "bf16" else y
    tok = w["tokens"].to_numpy().ravel()[:rows_sample].astype(np.int64)
    reps, t = 0, 0.0
    while reps < 1 or (t < min_seconds and reps < 1000):
        t0 = time.perf_counter()
        z = O.tempered(x, w["temperature"], keep=keep)
        O.token_logp(z, tok)
        O.entropy(z)
        if y is not None:
            r = O.tempered(y, w["temperature"], keep=keep)
            O.token_logp(r, tok)
            O.kl(z, r)
        t += time.perf_counter() - t0
        reps += 1
    return {"value": reps * rows_sample / t, "unit": "rows/s", "cores": 1, "kind": "port", "cpu": cpu_model(),
            "sample": f"{reps} x {rows_sample} {w['name']} rows (V={V}): the oracle's f64 scoring restatement "
                      f"(tempered values, log-softmax gather, {'exact KL, ' if y is not None else ''}entropy), "
                      f"single thread, {t:.2f} s"}


CACHE_BYTES = 1 << 30  # inputs cycled per launch: 4x the 256 MB Infinity Cache, so every read is from HBM


def bench_sample(nr, W, args, name):
    """c4 (the north star) or c2: one launch of nt_hip_rl_sample per step.

    A launch reads 98 MB at c4 (8 MB at c2), which the 256 MB Infinity Cache (MALL) in front of
    HBM would hold from one launch to the next. So the timed launches cycle over enough
    independently generated copies of the inputs (at least 1 GiB in all) that each launch's
    input was last touched a GiB of traffic earlier: `value` and `roofline` are HBM-cold. The
    same launches on one input, re-read every time (cache-warm, as when the logits were just
    written by the readout), are reported beside them as `warm_cache`."""
    shared = name == "c4s"  # C4 with one grammar mask [1, V] shared by every row (mask_ld 0)
    f32mask = name == "c4f"  # C4's grammar mask as the reference's f32 additive 0 / -inf mask

    def mk_w(sd):
        if name == "c2":
            return W.c2(sd)
        w = W.c4(sd, shared_mask=shared)
        if f32mask:
            keep = w["mask"].to_numpy()
            w["mask_f32"] = nr.Tensor.from_numpy(np.where(keep != 0, 0.0, -np.inf).astype(np.float32))
        return w

    w = mk_w(args.seed)
    rows, V = w["rows"], w["V"]
    dt = nr.NT_BF16 if w["logits"].dtype == "bf16" else nr.NT_F32
    mk = nr.NT_MASK_F32 if f32mask else (nr.NT_MASK_U8 if w["mask"] is not None else nr.NT_MASK_NONE)
    mkey = "mask_f32" if f32mask else "mask"
    esz = 2 if dt == nr.NT_BF16 else 4
    # Algorithmic bytes per launch: every input read once, every output written once.
    mask_row = 4 * V if f32mask else (V if (mk == nr.NT_MASK_U8 and not shared) else 0)
    per_row = esz * V + mask_row + 8 + 4 + 4 + 1  # logits, mask, uniform, id, logp, status
    bytes_launch = per_row * rows + (V if shared else 0)
    copies = max(2, -(-CACHE_BYTES // bytes_launch))
    ws = [w] + [mk_w(args.seed + 1 + k) for k in range(copies - 1)]
    n_launch = args.warmup + args.steps
    U = nr.Tensor.from_numpy(nr.Rng(args.seed, f"{name}/uniforms").uniforms(rows * n_launch), "f64")
    ids = nr.IntTensor((rows,))
    logp = nr.Tensor((rows,), "f32")
    status = nr.Tensor((rows,), "u8")
    L = nr.lib()

    def argv_for(pick):
        out = []
        for i in range(n_launch):
            x = pick(i)
            out.append(nr.NtRlSampleArgs(x["logits"].ptr, dt, mk, rows, V, V,
                                         x[mkey].ptr if x["mask"] is not None else None,
                                         V if (x["mask"] is not None and not shared) else 0, w["temperature"],
                                         U.ptr + 8 * rows * i,
                                         ids.ptr, logp.ptr, None, status.ptr))
        return out

    cold = argv_for(lambda i: ws[i % copies])
    warm = argv_for(lambda i: w)
    nr._check(L.nt_hip_rl_sample(C.byref(cold[0])), "sample")
    warm_s = clock_warmup(nr, lambda i: L.nt_hip_rl_sample(C.byref(cold[i % len(cold)])), args.clock_warmup)
    ms, wall = timed(nr, args.steps, args.warmup, lambda i: L.nt_hip_rl_sample(C.byref(cold[i])))
    st = status.to_numpy()
    if np.any(st != 0):
        raise SystemExit(f"bench: {int(np.sum(st != 0))} rows refused")
    ms_warm, _ = timed(nr, args.steps, args.warmup, lambda i: L.nt_hip_rl_sample(C.byref(warm[i])))
    # More repetitions of the same K cold launches, outside the contract's timed region: the spread
    # of the per-launch average from one K-launch window to the next.
    repeats = [timed(nr, args.steps, 0, lambda i: L.nt_hip_rl_sample(C.byref(cold[i])))[0] for _ in range(5)]
    # One launch on copy 0 with the first uniforms, for the parity check of the CPU leg.
    nr._check(L.nt_hip_rl_sample(C.byref(cold[0])), "sample")
    gpu_out = (ids.to_numpy().ravel().astype(np.int64), logp.to_numpy().ravel().copy(),
               U.to_numpy().ravel()[:rows].copy())
    roof = roofline(bytes_launch, ms, "k_sample_rq_c4_traffic.json" if name == "c4" else None)
    roof["inputs"] = (f"HBM-cold: launches cycle over {copies} input copies "
                      f"({copies * bytes_launch / 2**20:.0f} MiB), beyond the 256 MB Infinity Cache")
    roof["warm_cache"] = {"ms": ms_warm, "achieved": bytes_launch / (ms_warm * 1e-3) / 1e9,
                          "frac": bytes_launch / (ms_warm * 1e-3) / 1e9 / HBM_PEAK_GBS,
                          "inputs": "one input re-read every launch (served partly by the Infinity Cache)"}
    if name == "c4":
        roof["measured_copy_gbs"] = copy_peak(nr)  # a device-to-device copy on this box, for scale
        roof["practical"] = practical_floor(nr, bytes_launch, roof.get("traffic"), ms, rows)
    if name == "c4f":
        metric = "rows/sec + achieved HBM GB/s, fused masked sample+logprob, V=128256 bf16, f32 additive mask"
        config = {"workload": "c4 under the reference's own mask form: bf16 logits [1,256,1,128256] ~ N(0,2^2), the "
                              "runs grammar mask as an f32 additive 0 / -inf mask [256,V] (4 bytes a token), temperature "
                              "0.7, fused sample + logp; launches cycle over independent input copies (1 GiB in all)",
                  "rows": rows, "vocab": V, "parallelism": "none (1 GPU)"}
    elif name == "c4s":
        metric = "rows/sec + achieved HBM GB/s, fused masked sample+logprob, V=128256 bf16, one shared mask"
        config = {"workload": "c4 with one u8 grammar mask [1,V] shared by the 256 rows (mask_ld 0): bf16 logits "
                              "[1,256,1,128256] ~ N(0,2^2), temperature 0.7, fused sample + logp; launches cycle over "
                              "independent input copies (1 GiB in all)", "rows": rows, "vocab": V,
                  "parallelism": "none (1 GPU)"}
    elif name == "c4":
        metric = "rows/sec + achieved HBM GB/s, fused masked sample+logprob, V=128256 bf16"
        config = {"workload": "c4 constrained decode: bf16 logits [1,256,1,128256] ~ N(0,2^2), u8 grammar mask "
                              "[256,V] of contiguous runs (~30% kept), temperature 0.7, fused sample + logp; launches cycle over "
                              "independent input copies (1 GiB in all) so every read comes from HBM",
                  "rows": rows, "vocab": V, "parallelism": "none (1 GPU)"}
    else:
        metric = "rows/sec + achieved HBM GB/s, fused sample+logprob, V=32000 f32 (decode step)"
        config = {"workload": "c2 decode step: f32 logits [1,64,1,32000] ~ N(0,1) + 8 spikes of +6 per row, no mask, "
                              "temperature 0.8, fused sample + logp; launches cycle over independent input copies (1 GiB in "
                              "all) so every read comes from HBM", "rows": rows, "vocab": V,
                  "parallelism": "none (1 GPU)"}
    out = line(metric, rows / (ms * 1e-3), args.steps, args.warmup, ms, "bf16" if esz == 2 else "f32", config, roof,
               achieved_gbs=roof["achieved"], wall_s_timed_region=wall, key=nr.key(),
               ms_per_step_repeats=repeats, ms_per_step_median_of_repeats=float(np.median(repeats)),
               clock_warmup_s=round(warm_s, 3))
    if args.cpu_rows > 0:
        n_cpu = min(args.cpu_rows, rows)
        gpu = tuple(a[:n_cpu] for a in gpu_out)
        out["cpu_baseline"] = cpu_baseline(w, n_cpu, args.seed, args.cpu_seconds, gpu=gpu)
        # the GPU launch's parity against the oracle (checked beside the CPU leg, outside every
        # timed region) is the line's own object
        if "parity" in out["cpu_baseline"]:
            out["parity"] = out["cpu_baseline"].pop("parity")
    return out


def bench_gumbel(nr, W, args):
    """c4g: the reference's own sampler, Gumbel-max sample_categorical (rl.rs:488-529), at C4's
    shape on the device: one launch of nt_hip_rl_sample_gumbel per step, each draw's u64 generated
    where it is used (ChaCha20 at the stream's word position, one u64 per logit in row-major
    order), each launch at its own position of one stream. Inputs cycle over the same HBM-cold
    copies as c4. The CPU baseline is the same op sequence on Cpu(Reference) and Cpu(Fast)."""
    from oracle import oracle as O
    w = W.c4(args.seed)
    rows, V = w["rows"], w["V"]
    per_row = 2 * V + V + 4 + 1  # logits, mask, id, status (the draws are generated, not read)
    bytes_launch = per_row * rows
    copies = max(2, -(-CACHE_BYTES // bytes_launch))
    ws = [w] + [W.c4(args.seed + 1 + k) for k in range(copies - 1)]
    rng = nr.Rng(args.seed, "c4g/stream")
    key = rng.key()
    block0, word0 = rng.word_pos()
    blocks_per_launch = rows * V // 8  # one u64 per logit, eight to a 64-byte keystream block
    ids, st = nr.IntTensor((rows,)), nr.Tensor((rows,), "u8")
    L = nr.lib()

    def argv(x, i):
        return nr.NtRlGumbelArgs(x["logits"].ptr, nr.NT_BF16, nr.NT_MASK_U8, rows, V, V, x["mask"].ptr, V,
                                 w["temperature"], key, block0 + i * blocks_per_launch, word0, 0, ids.ptr, st.ptr)

    n_launch = args.warmup + args.steps
    cold = [argv(ws[i % copies], i) for i in range(n_launch)]
    warm = [argv(w, i) for i in range(n_launch)]
    nr._check(L.nt_hip_rl_sample_gumbel(C.byref(cold[0])), "sample_gumbel")
    warm_s = clock_warmup(nr, lambda i: L.nt_hip_rl_sample_gumbel(C.byref(cold[i % len(cold)])), args.clock_warmup)
    ms, wall = timed(nr, args.steps, args.warmup, lambda i: L.nt_hip_rl_sample_gumbel(C.byref(cold[i])))
    if np.any(st.to_numpy() != 0):
        raise SystemExit("bench c4g: refused rows")
    ms_warm, _ = timed(nr, args.steps, args.warmup, lambda i: L.nt_hip_rl_sample_gumbel(C.byref(warm[i])))
    # parity, outside the timed regions: launch 0 (copy 0, the stream's start) against the
    # oracle's Cpu(Reference) op sequence on the same stream, for the first rows
    nr._check(L.nt_hip_rl_sample_gumbel(C.byref(cold[0])), "sample_gumbel")
    n_par = min(32, rows)
    dev = ids.to_numpy().ravel()[:n_par].astype(np.int64)
    x = W.bf16_to_f32(w["logits"].to_numpy().reshape(rows, V)[:n_par])
    keep = w["mask"].to_numpy().reshape(rows, V)[:n_par]
    cpu = O.cpuref_sample_gumbel(x, w["temperature"], O.Rng(args.seed, "c4g/stream"), keep=keep)
    hbm = roofline(bytes_launch, ms)
    roof = valu_roofline(nr, ms, "k_sample_gumbel_c4_valu.json")
    roof["hbm"] = {"achieved": hbm["achieved"], "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": hbm["frac"],
                   "algorithmic_bytes_per_launch": bytes_launch,
                   "inputs": (f"HBM-cold: launches cycle over {copies} input copies "
                              f"({copies * bytes_launch / 2**20:.0f} MiB), beyond the 256 MB Infinity Cache")}
    roof["note"] = ("bound by generating the draws (a ChaCha20 block per 8 logits holding an allowed one, and "
                    "two f32 hardware logarithms per allowed logit; f64 only where a row has several "
                    "candidates): the VALU instruction count, not HBM")
    roof["warm_cache"] = {"ms": ms_warm, "achieved_hbm": bytes_launch / (ms_warm * 1e-3) / 1e9,
                          "frac_hbm": bytes_launch / (ms_warm * 1e-3) / 1e9 / HBM_PEAK_GBS}
    config = {"workload": "c4 rows through the reference's Gumbel-max sample_categorical: bf16 logits "
                          "[1,256,1,128256] ~ N(0,2^2), u8 grammar mask of contiguous runs (~30% kept), temperature "
                          "0.7, one u64 of the caller's ChaCha20 stream per logit; launches cycle over independent "
                          "input copies (1 GiB in all)", "rows": rows, "vocab": V, "parallelism": "none (1 GPU)"}
    out = line("rows/sec, the reference's Gumbel-max sample_categorical at c4's shape (V=128256 bf16, u8 mask)",
               rows / (ms * 1e-3), args.steps, args.warmup, ms, "bf16", config, roof, wall_s_timed_region=wall,
               key=nr.key(), clock_warmup_s=round(warm_s, 3),
               parity={"rows": n_par, "ids_differ_from_cpuref": int(np.sum(dev != cpu)),
                       "what": "device draws against Cpu(Reference)'s op sequence for the same stream"})
    if args.cpu_rows > 0:
        out["cpu_baseline"] = cpu_baseline(w, min(args.cpu_rows, rows), args.seed, args.cpu_seconds)
    return out


def bench_score(nr, W, args, name):
    """c3 or c5: one fused scoring launch per step plus the small per-token follow-ups."""
    w = W.c3(args.seed) if name == "c3" else W.c5(args.seed)
    rows, V = w["rows"], w["V"]
    shp = w["logits"].shape[:-1]
    L = nr.lib()
    dt = nr.NT_BF16 if w["logits"].dtype == "bf16" else nr.NT_F32
    esz = 2 if dt == nr.NT_BF16 else 4
    out_t = lambda: nr.Tensor(shp, "f32")
    lp, ent, status = out_t(), out_t(), nr.Tensor(shp, "u8")
    ref = w.get("ref")
    rlp, kl, k3 = (out_t(), out_t(), out_t()) if ref is not None else (None, None, None)
    mask = w.get("mask")
    a = nr.NtRlScoreArgs(w["logits"].ptr, ref.ptr if ref is not None else None, dt,
                         nr.NT_MASK_U8 if mask is not None else nr.NT_MASK_NONE, rows, V, V,
                         mask.ptr if mask is not None else None, V if mask is not None else 0, w["temperature"],
                         w["tokens"].ptr, lp.ptr, rlp.ptr if rlp else None, kl.ptr if kl else None, ent.ptr,
                         status.ptr)
    score = lambda i: L.nt_hip_rl_score(C.byref(a))
    nr._check(score(0), "score")
    # the dominant kernel alone, for the roofline
    ms_score, _ = timed(nr, args.steps, args.warmup, score)
    # logits (x2 with a reference), mask, token, logp, entropy, status (+ reference logp, KL)
    per_row = (2 if ref is not None else 1) * esz * V + (V if mask is not None else 0) + 4 + 4 + 4 + 1
    if ref is not None:
        per_row += 4 + 4
    bytes_score = per_row * rows
    if name == "c3":
        def step(i):
            score(i)
            nr._check(L.nt_hip_rl_kl_estimate(lp.ptr, rlp.ptr, None, rows, int(nr.KlEstimator.K3), 0.0, k3.ptr),
                      "kl_estimate")
    else:
        S, B, T = shp
        seq = nr.Tensor((S, B), "f32")

        adv = nr.Tensor((S, B), "f32")

        def step(i):
            score(i)
            nr._check(L.nt_hip_rl_reduce_tokens(lp.ptr, None, S, B, T, int(nr.TokenReduction.PER_SEQUENCE), seq.ptr),
                      "reduce_tokens")
            # group-relative advantages over groups of 8 along B (rl.rs:416-469), on the device
            nr._check(L.nt_hip_rl_group_advantages(seq.ptr, S * B // 8, 8, 1, 1e-6, 1, adv.ptr), "group_advantages")
    ms, wall = timed(nr, args.steps, args.warmup, step)
    st = status.to_numpy()
    if np.any(st != 0):
        raise SystemExit(f"bench: {int(np.sum(st != 0))} rows refused")
    roof = roofline(bytes_score, ms_score, f"k_score_{name}_traffic.json")
    roof["kernel"] = "k_score"
    roof["kernel_ms"] = ms_score
    if name == "c3":
        metric = "rows/sec + achieved HBM GB/s, fused PPO scoring (logp, ref logp, exact KL, k3, entropy), V=50304 bf16"
        config = {"workload": "c3 PPO scoring: bf16 policy [8,16,512,50304] ~ N(0,1.5^2), reference = policy + "
                              "N(0,0.1^2) (RNE), tokens uniform; logp, ref logp, exact KL, entropy, k3",
                  "rows": rows, "vocab": V, "parallelism": "none (1 GPU)"}
    else:
        metric = ("rows/sec + achieved HBM GB/s, fused masked scoring (logp, entropy) + group advantages, "
                  "V=151936 f32")
        config = {"workload": "c5 rollout scoring: f32 [4,32,1024,151936] ~ N(0,1) + Zipf(1.1) rank bias, u8 mask "
                              "Bernoulli(0.9); logp, entropy, per-sequence mean logp, group advantages (8 along B)",
                  "rows": rows, "vocab": V, "parallelism": "none (1 GPU)"}
    out = line(metric, rows / (ms * 1e-3), args.steps, args.warmup, ms, "bf16" if esz == 2 else "f32", config, roof,
               achieved_gbs=roof["achieved"], wall_s_timed_region=wall, key=nr.key())
    if args.cpu_rows > 0:
        out["cpu_baseline"] = cpu_baseline_scoring(w, min(args.cpu_rows, 64), args.cpu_seconds)
    return out


def bench_score_grad(nr, W, args):
    """c3b: the c3 PPO step's scoring forward (nt_hip_rl_score with the per-row log-sum-exp saved)
    and its fused backward (nt_hip_rl_score_backward: d(g_logp logp + g_kl KL + g_H H)/d logits,
    written in the logits' dtype), one of each per step."""
    w = W.c3(args.seed)
    rows, V = w["rows"], w["V"]
    shp = w["logits"].shape[:-1]
    L = nr.lib()
    out_t = lambda: nr.Tensor(shp, "f32")
    lp, rlp, kl, ent, status = out_t(), out_t(), out_t(), out_t(), nr.Tensor(shp, "u8")
    lb, lr, rlb, rlr = out_t(), out_t(), out_t(), out_t()
    a = nr.NtRlScoreArgs(w["logits"].ptr, w["ref"].ptr, nr.NT_BF16, nr.NT_MASK_NONE, rows, V, V, None, 0,
                         w["temperature"], w["tokens"].ptr, lp.ptr, rlp.ptr, kl.ptr, ent.ptr, status.ptr, lb.ptr,
                         lr.ptr, rlb.ptr, rlr.ptr)
    # upstream gradients of a GRPO-style loss: advantages on logp, beta = 0.04 on KL, -0.01 on entropy
    rng = np.random.default_rng(args.seed)
    g_lp = nr.Tensor.from_numpy(rng.normal(0, 1, shp).astype(np.float32))
    g_kl = nr.Tensor.from_numpy(np.full(shp, 0.04, np.float32))
    g_h = nr.Tensor.from_numpy(np.full(shp, -0.01, np.float32))
    grad = nr.Tensor(w["logits"].shape, "bf16")
    b = nr.NtRlScoreGradArgs(w["logits"].ptr, w["ref"].ptr, nr.NT_BF16, nr.NT_MASK_NONE, rows, V, V, None, 0,
                             w["temperature"], w["tokens"].ptr, lb.ptr, lr.ptr, rlb.ptr, rlr.ptr, kl.ptr, ent.ptr,
                             g_lp.ptr, g_kl.ptr, g_h.ptr, grad.ptr, nr.NT_BF16, 0, V)
    fwd = lambda i: L.nt_hip_rl_score(C.byref(a))
    bwd = lambda i: L.nt_hip_rl_score_backward(C.byref(b))
    nr._check(fwd(0), "score")
    nr._check(bwd(0), "score backward")
    if np.any(status.to_numpy() != 0):
        raise SystemExit("bench: refused rows")
    ms_bwd, _ = timed(nr, args.steps, args.warmup, bwd)
    ms, wall = timed(nr, args.steps, args.warmup, lambda i: (fwd(i), bwd(i)))
    # backward, per row: policy and reference logits read, the gradient written (bf16), and the
    # token, four log-sum-exp values, KL, entropy and three upstream gradients read
    bytes_bwd = rows * (2 * 2 * V + 2 * V + 4 + 4 * 4 + 4 + 4 + 3 * 4)
    roof = roofline(bytes_bwd, ms_bwd, "k_score_grad_c3b_traffic.json")
    roof["kernel"] = "k_score_grad"
    roof["kernel_ms"] = ms_bwd
    metric = "rows/sec + achieved HBM GB/s, fused PPO scoring forward + backward (logp, KL, entropy), V=50304 bf16"
    config = {"workload": "c3b PPO scoring forward and backward: bf16 policy + reference [8,16,512,50304] as c3; "
                          "forward logp, ref logp, exact KL, entropy; backward d(g_logp logp + 0.04 KL - 0.01 H)/d "
                          "logits in bf16, g_logp ~ N(0,1)", "rows": rows, "vocab": V, "parallelism": "none (1 GPU)"}
    out = line(metric, rows / (ms * 1e-3), args.steps, args.warmup, ms, "bf16", config, roof,
               achieved_gbs=roof["achieved"], wall_s_timed_region=wall, key=nr.key())
    if args.cpu_rows > 0:
        out["cpu_baseline"] = cpu_baseline_score_grad(w, min(args.cpu_rows, 16), args.cpu_seconds)
    return out


def cpu_baseline_score_grad(w, rows_sample, min_seconds=10.0):
    """The oracle's forward statistics and f64 gradient of a bounded row sample on one host core."""
    import workloads as W
    from oracle import oracle as O
    V = w["V"]
    x = W.bf16_to_f32(W.download_rows(w["logits"], range(rows_sample), V))
    y = W.bf16_to_f32(W.download_rows(w["ref"], range(rows_sample), V))
    tok = w["tokens"].to_numpy().ravel()[:rows_sample].astype(np.int64)
    g_lp = np.random.default_rng(1).normal(0, 1, rows_sample)
    reps, t = 0, 0.0
    while reps < 1 or (t < min_seconds and reps < 1000):
        t0 = time.perf_counter()
        O.token_logp(x, tok)
        O.token_logp(y, tok)
        O.score_grad(x, tok, y, g_lp, np.full(rows_sample, 0.04), np.full(rows_sample, -0.01))
        t += time.perf_counter() - t0
        reps += 1
    return {"value": reps * rows_sample / t, "unit": "rows/s", "cores": 1, "kind": "port", "cpu": cpu_model(),
            "sample": f"{reps} x {rows_sample} c3 rows (V={V}): the oracle's f64 forward (logp, ref logp) and "
                      f"gradient of g_logp logp + 0.04 KL - 0.01 H (row statistics, KL, entropy, then each "
                      f"element), single thread, {t:.2f} s"}


def bench_ops(nr, args):
    """The general device ops (include/noetic_ops.h) at C4's shape, [256, 128256]: each op's
    HIP-event time per call through the C ABI (outputs allocated before timing) and its
    algorithmic bytes (every input element read once, every output element written once) against
    the HBM peak. Rows are f32 unless named."""
    from noetic_ops import BinaryOp, Layout, ReduceOp, UnaryOp

    rows, V = 256, 128256
    L = nr.lib()
    rng = np.random.default_rng(args.seed)
    xf = rng.normal(0, 2, (rows, V)).astype(np.float32)
    x = nr.Tensor.from_numpy(xf)
    xb = nr.Tensor.from_numpy((xf.view(np.uint32) >> 16).astype(np.uint16), "bf16")
    mask = nr.Tensor.from_numpy(np.where(rng.random((1, V)) < 0.3, 0.0, -np.inf).astype(np.float32))
    idx = nr.Tensor.from_numpy(rng.integers(0, V, (rows, 1)).astype(np.int32))
    y = nr.Tensor((rows, V), "f32")
    yr = nr.Tensor((rows,), "f32")
    yi = nr.Tensor((rows, V), "i32")
    n = rows * V
    lay = Layout([rows, V]).c()
    mlay = Layout([1, V]).broadcast([rows, V]).c()
    tlay = Layout([V, rows], [1, V]).c()
    P = lambda t: C.c_void_p(t.ptr)
    ck = lambda rc: nr._check(rc, "op")
    cases = {
        "cast bf16->f32": (lambda: ck(L.nt_hip_cast(P(xb), C.byref(lay), 1, 0, P(y))), 6 * n),
        "unary div_scalar": (lambda: ck(L.nt_hip_unary(int(UnaryOp.DIV_SCALAR), 0.7, P(x), C.byref(lay), P(y))), 8 * n),
        "unary exp": (lambda: ck(L.nt_hip_unary(int(UnaryOp.EXP), 0.0, P(x), C.byref(lay), P(y))), 8 * n),
        "binary add [1,V] mask": (lambda: ck(L.nt_hip_binary(int(BinaryOp.ADD), P(x), C.byref(lay), P(mask),
                                                             C.byref(mlay), P(y))), 8 * n + 4 * V),
        "copy transposed [V,rows]": (lambda: ck(L.nt_hip_copy(P(x), C.byref(tlay), 4, P(y))), 8 * n),
        "reduce_dim sum last axis (CpuRef order)": (lambda: ck(L.nt_hip_reduce_dim(int(ReduceOp.SUM), P(x), rows, V, 1,
                                                                                   1, P(yr))), 4 * n + 4 * rows),
        "reduce_dim argmax last axis": (lambda: ck(L.nt_hip_reduce_dim(int(ReduceOp.ARGMAX), P(x), rows, V, 1, 1,
                                                                       P(yr))), 4 * n + 4 * rows),
        "gather token logits": (lambda: ck(L.nt_hip_gather(P(x), rows, V, 1, P(idx), 1, P(yr))), 12 * rows),
        # read each value once, write each value and its I32 position once (the runs and merge
        # passes in between are the sort's own traffic)
        "sort_desc of every row (top-p's sort)": (lambda: ck(L.nt_hip_sort_desc(P(x), rows, V, 1, P(y), P(yi))),
                                                  12 * n),
    }
    res = {}
    steps, warmup = min(args.steps, 50), min(args.warmup, 5)
    for name, (fn, nbytes) in cases.items():
        ms, _ = timed(nr, steps, warmup, lambda i: fn())
        gbs = nbytes / (ms * 1e-3) / 1e9
        res[name] = {"us": round(ms * 1e3, 2), "bytes": nbytes, "gbs": round(gbs, 1),
                     "frac": round(gbs / HBM_PEAK_GBS, 4)}
    top = res["unary div_scalar"]
    return {"metric": "general device ops at [256,128256]: HIP-event time and achieved HBM GB/s per op",
            "value": top["gbs"], "unit": "GB/s (unary div_scalar)", "n_gpus": 1, "steps": steps, "warmup": warmup,
            "ms_per_step": top["us"] / 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "f32", "data": "synthetic",
            "config": {"workload": "ops: the GpuBackend general ops on C4's shape, f32 rows unless named"},
            "ops": res}


VALU_F32_PEAK_TFLOPS = 78.6  # 256 CUs x 4 SIMDs x 16 lanes x 2 flops x 2.4 GHz, one v_fma_f32 per lane


def bench_matmul(nr, args):
    """nt_hip_matmul (GpuBackend::matmul, CpuRef's fma-chain order bit for bit) at the reference's
    matmul_throughput shapes (src/tensor/tests/gpu/kernels.rs:262-291: A.B 1024^3, A.B 512x512x2048,
    A.B^T 512x2048x512, A^T.B 512x512x2048) and at 4096^3, on resident f32 operands. The order
    rules out the matrix cores, so the roofline is the VALU's f32 fma rate without packed
    instructions (78.6 TFLOP/s)."""
    from noetic_ops import Layout
    L = nr.lib()
    P = lambda t: C.c_void_p(t.ptr)  # noqa: E731
    rng = np.random.default_rng(args.seed)
    cases = [("A.B 1024^3", 1024, 1024, 1024, False, False), ("A.B 512x512x2048", 512, 2048, 512, False, False),
             ("A.B^T 512x2048x512", 512, 512, 2048, False, True), ("A^T.B 512x512x2048", 512, 2048, 512, True, False),
             ("A.B 4096^3", 4096, 4096, 4096, False, False)]
    res = {}
    steps, warmup = min(args.steps, 20), min(args.warmup, 3)
    for name, m, k, n, ta, tb in cases:
        a = nr.Tensor.from_numpy(rng.uniform(-2, 2, (k, m) if ta else (m, k)).astype(np.float32))
        b = nr.Tensor.from_numpy(rng.uniform(-2, 2, (n, k) if tb else (k, n)).astype(np.float32))
        al = Layout([k, m]).swapped(0, 1) if ta else Layout([m, k])
        bl = Layout([n, k]).swapped(0, 1) if tb else Layout([k, n])
        y = nr.Tensor((m, n), "f32")
        ca, cb = al.c(), bl.c()
        ck = lambda rc: nr._check(rc, "matmul")  # noqa: E731
        ms, _ = timed(nr, steps, warmup, lambda i: ck(L.nt_hip_matmul(P(a), C.byref(ca), P(b), C.byref(cb), P(y))))
        tf = 2.0 * m * k * n / (ms * 1e-3) / 1e12
        res[name] = {"ms": round(ms, 4), "tflops": round(tf, 2), "frac_of_valu_peak": round(tf / VALU_F32_PEAK_TFLOPS, 4)}
        if name in ("A.B 1024^3", "A.B 4096^3"):
            ms, _ = timed(nr, steps, warmup,
                          lambda i: ck(L.nt_hip_matmul_half(P(a), C.byref(ca), P(b), C.byref(cb), P(y))))
            tf = 2.0 * m * k * n / (ms * 1e-3) / 1e12
            res["half " + name] = {"ms": round(ms, 4), "tflops": round(tf, 2),
                                   "frac_of_bf16_mfma_peak": round(tf / 2500.0, 4)}
    top = res["A.B 4096^3"]
    out = {"metric": "f32 matmul (CpuRef's arithmetic bit for bit) TFLOP/s", "value": top["tflops"],
           "unit": "TFLOP/s (A.B 4096^3)", "n_gpus": 1, "steps": steps, "warmup": warmup,
           "ms_per_step": top["ms"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "f32", "data": "synthetic",
           "config": {"workload": "matmul: uniform(-2, 2) f32 operands resident on the device, fresh-output-free "
                                  "(one preallocated output per shape)"},
           "roofline": {"bound": "valu", "achieved": top["tflops"], "peak": VALU_F32_PEAK_TFLOPS, "unit": "TFLOP/s",
                        "frac": top["frac_of_valu_peak"], "traffic": None,
                        "note": "the published 157.3 TFLOP/s f32 figure counts matrix-core or packed-f32 "
                                "instructions; neither keeps the reference's per-output fma chain"},
           "shapes": res}
    if args.cpu_rows > 0:
        import time as _t
        from oracle import oracle as O
        a = rng.uniform(-2, 2, (64, 1024)).astype(np.float32)
        b = rng.uniform(-2, 2, (1024, 1024)).astype(np.float32)
        reps, t_ref = 0, 0.0
        while reps < 1 or (t_ref < args.cpu_seconds and reps < 100):
            t0 = _t.perf_counter()
            O.matmul(a, b)
            t_ref += _t.perf_counter() - t0
            reps += 1
        out["cpu_baseline"] = {"value": reps * 2.0 * 64 * 1024 * 1024 / t_ref / 1e12, "unit": "TFLOP/s", "cores": 1,
                               "kind": "port", "cpu": cpu_model(),
                               "sample": f"{reps} x [64,1024]x[1024,1024] through oracle.c's fmaf chains, one thread"}
    return out


def bench_readout(nr, W, args):
    """One decode step at C4's shape with the readout: logits[256, 128256] = h[256, 4096] . W in
    bf16, then the masked inverse-CDF sample + log-prob (u8 C4 mask, tau 0.7).

    Fused (the value): nt_hip_rl_readout_sample, the product and the sampler's row records in one
    MFMA kernel and a per-row resolve, the logits never written; the weight packed once from the
    reference's [d, V] Linear layout into the matrix cores' fragment order (timed separately, as a
    loader would run it once).
    Unfused (beside it): torch.matmul (hipBLASLt) into bf16 logits, then nt_hip_rl_sample on
    them, with the weight in the reference's [d, V] layout and in the vocabulary-major one.
    Scoring (`score`, beside it): nt_hip_rl_readout_score (the log-probability of each row's drawn
    token and the entropy, the logits never written) against hipBLASLt's GEMM and nt_hip_rl_score
    on the bf16 logits."""
    import torch

    rows, d, V = 256, 4096, 128256
    stream = C.c_void_p()
    nr._check(nr.lib().nt_hip_stream(C.byref(stream)), "stream")
    ts = torch.cuda.ExternalStream(stream.value, device="cuda:0")
    g = torch.Generator(device="cuda:0").manual_seed(args.seed)
    w = W.c4(args.seed)
    with torch.cuda.stream(ts):
        h = torch.randn(rows, d, device="cuda:0", dtype=torch.bfloat16, generator=g)
        w_vd = (torch.randn(V, d, device="cuda:0", dtype=torch.bfloat16, generator=g) * (2.0 / 64.0)).to(torch.bfloat16)
        logits = torch.empty(rows, V, device="cuda:0", dtype=torch.bfloat16)
    torch.cuda.synchronize()
    # the reference's layout [d, V], made once by the library's own transposing copy (what a
    # loader would run once, the other way)
    L = nr.lib()
    w_dv = torch.empty(d, V, device="cuda:0", dtype=torch.bfloat16)
    lay = nr.NtLayout()
    lay.rank, lay.offset = 2, 0
    lay.shape[0], lay.shape[1] = d, V
    lay.strides[0], lay.strides[1] = 1, d  # the [V, d] buffer read as its [d, V] transpose
    t0 = time.perf_counter()
    nr._check(L.nt_hip_copy(C.c_void_p(w_vd.data_ptr()), C.byref(lay), 2, C.c_void_p(w_dv.data_ptr())), "transpose")
    nr.sync()
    transpose_s = time.perf_counter() - t0
    nbytes = int(L.nt_hip_rl_readout_packed_bytes(V, d))
    w_packed = torch.empty(nbytes, device="cuda:0", dtype=torch.uint8)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    nr._check(L.nt_hip_rl_readout_pack_weight(C.c_void_p(w_dv.data_ptr()), nr.NT_BF16, nr.NT_READOUT_W_DV, V, d, V,
                                              C.c_void_p(w_packed.data_ptr())), "pack")
    nr.sync()
    pack_s = time.perf_counter() - t0
    U = nr.Tensor.from_numpy(nr.Rng(args.seed, "readout/uniforms").uniforms(rows), "f64")
    ids, logp, st = nr.IntTensor((rows,)), nr.Tensor((rows,), "f32"), nr.Tensor((rows,), "u8")
    a = nr.NtRlSampleArgs(logits.data_ptr(), nr.NT_BF16, nr.NT_MASK_U8, rows, V, V, w["mask"].ptr, V, 0.7, U.ptr,
                          ids.ptr, logp.ptr, None, st.ptr)
    ids2, logp2, st2 = nr.IntTensor((rows,)), nr.Tensor((rows,), "f32"), nr.Tensor((rows,), "u8")
    fa = nr.NtRlReadoutSampleArgs(h.data_ptr(), w_packed.data_ptr(), rows, V, d, d, nr.NT_MASK_U8, nr.NT_BF16,
                                  w["mask"].ptr, V, 0.7, U.ptr, ids2.ptr, logp2.ptr, st2.ptr, None, None, None)

    def fused(i):
        nr._check(L.nt_hip_rl_readout_sample(C.byref(fa)), "readout sample")

    # scoring the drawn tokens (ids2, the fused step's draws): fused, and on the written logits
    slp, sent, sst = nr.Tensor((rows,), "f32"), nr.Tensor((rows,), "f32"), nr.Tensor((rows,), "u8")
    sa = nr.NtRlReadoutScoreArgs(h.data_ptr(), w_packed.data_ptr(), rows, V, d, d, nr.NT_MASK_U8, nr.NT_BF16,
                                 w["mask"].ptr, V, 0.7, ids2.ptr, slp.ptr, sent.ptr, sst.ptr, None)
    ulp, uent, ust = nr.Tensor((rows,), "f32"), nr.Tensor((rows,), "f32"), nr.Tensor((rows,), "u8")
    ua = nr.NtRlScoreArgs(logits.data_ptr(), None, nr.NT_BF16, nr.NT_MASK_U8, rows, V, V, w["mask"].ptr, V, 0.7,
                          ids2.ptr, ulp.ptr, None, None, uent.ptr, ust.ptr, None, None, None, None)

    def fused_score(i):
        nr._check(L.nt_hip_rl_readout_score(C.byref(sa)), "readout score")

    def score_on_logits(i):
        nr._check(L.nt_hip_rl_score(C.byref(ua)), "score")

    def gemm_dv(i):
        with torch.cuda.stream(ts):
            torch.matmul(h, w_dv, out=logits)

    def gemm_vd(i):
        with torch.cuda.stream(ts):
            torch.matmul(h, w_vd.t(), out=logits)

    def sample(i):
        nr._check(L.nt_hip_rl_sample(C.byref(a)), "sample")

    def step_dv(i):
        gemm_dv(i)
        sample(i)

    def step_vd(i):
        gemm_vd(i)
        sample(i)

    def score_step_vd(i):
        gemm_vd(i)
        score_on_logits(i)

    steps, warmup = args.steps, args.warmup
    fused(0)
    warm_s = clock_warmup(nr, fused, args.clock_warmup)
    ms, wall = timed(nr, steps, warmup, fused)
    if np.any(st2.to_numpy() != 0):
        raise RuntimeError("readout: refused rows")
    # the unfused steps beside it: three interleaved rounds, medians
    res = {k: [] for k in ("fused", "gemm_dv", "gemm_vd", "sample", "step_dv", "step_vd", "fused_score", "score",
                           "score_step_vd")}
    for _ in range(3):
        res["fused"].append(timed(nr, steps, warmup, fused)[0])
        res["gemm_dv"].append(timed(nr, steps, warmup, gemm_dv)[0])
        res["gemm_vd"].append(timed(nr, steps, warmup, gemm_vd)[0])
        gemm_dv(0)
        res["sample"].append(timed(nr, steps, warmup, sample)[0])
        res["step_dv"].append(timed(nr, steps, warmup, step_dv)[0])
        res["step_vd"].append(timed(nr, steps, warmup, step_vd)[0])
        res["fused_score"].append(timed(nr, steps, warmup, fused_score)[0])
        gemm_vd(0)
        res["score"].append(timed(nr, steps, warmup, score_on_logits)[0])
        res["score_step_vd"].append(timed(nr, steps, warmup, score_step_vd)[0])
    med = {k: float(np.median(v)) * 1e3 for k, v in res.items()}
    if np.any(st.to_numpy() != 0):
        raise RuntimeError("readout: refused rows (unfused)")
    if np.any(sst.to_numpy() != 0) or np.any(ust.to_numpy() != 0):
        raise RuntimeError("readout: refused rows (scoring)")
    # the fused scorer against the unfused one on the same tokens (the unfused logits are bf16, the
    # fused f32: the difference is the logits' rounding, reported, not asserted)
    d_lp = float(np.max(np.abs(slp.to_numpy().astype(np.float64) - ulp.to_numpy())))
    d_ent = float(np.max(np.abs(sent.to_numpy().astype(np.float64) - uent.to_numpy())))
    w_bytes = V * d * 2
    step_bytes = w_bytes + rows * d * 2 + rows * V + rows * (8 + 4 + 4 + 1)
    flops = 2.0 * rows * d * V
    gbs = step_bytes / (ms * 1e-3) / 1e9
    tfs = flops / (ms * 1e-3) / 1e12
    roof = {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS,
            "traffic": None, "algorithmic_bytes_per_launch": step_bytes,
            "what": "the whole fused step (both launches) against the weight stream: the weight (1.05 GB) once, "
                    "h, the mask, the uniforms and the outputs",
            "mfma": {"achieved": tfs, "peak": 2500.0, "unit": "TFLOP/s", "frac": tfs / 2500.0,
                     "flops_per_step": flops}}
    return {"metric": "decode step at C4's shape: bf16 readout (h[256,4096] . W, V 128256) + masked sample + logprob",
            "value": rows / (ms * 1e-3), "unit": "rows/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
            "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic",
            "config": {"workload": "readout: nt_hip_rl_readout_sample, logits never written; weight [d, V] bf16 "
                                   "~ N(0, (2/64)^2) packed once, h ~ N(0,1), u8 C4 grammar mask, tau 0.7",
                       "rows": rows, "dim": d, "vocab": V},
            "roofline": roof, "wall_s_timed_region": wall,
            "unfused": {"fused_step_us_median_of_3": round(med["fused"], 2),
                        "hipblaslt_gemm_w_dv_us": round(med["gemm_dv"], 2),
                        "hipblaslt_gemm_w_vd_us": round(med["gemm_vd"], 2),
                        "sampler_on_bf16_logits_us": round(med["sample"], 2),
                        "gemm_plus_sampler_w_dv_us": round(med["step_dv"], 2),
                        "gemm_plus_sampler_w_vd_us": round(med["step_vd"], 2),
                        "speedup_vs_best_unfused": round(min(med["step_dv"], med["step_vd"]) / med["fused"], 3),
                        "note": "the unfused GEMM writes bf16 logits (hipBLASLt's output for bf16 operands); the "
                                "fused product keeps them in f32"},
            "score": {"what": "log-probability of each row's drawn token + entropy, same shape and mask",
                      "fused_readout_score_us": round(med["fused_score"], 2),
                      "score_on_bf16_logits_us": round(med["score"], 2),
                      "gemm_w_vd_plus_score_us": round(med["score_step_vd"], 2),
                      "speedup": round(med["score_step_vd"] / med["fused_score"], 3),
                      "max_abs_diff_logp_vs_bf16_logits": d_lp, "max_abs_diff_entropy_vs_bf16_logits": d_ent},
            "weight_transpose_once_s": round(transpose_s, 4), "weight_pack_once_s": round(pack_s, 4),
            "clock_warmup_s": round(warm_s, 3), "key": nr.key()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (default 200; 20 for c3/c5)")
    ap.add_argument("--warmup", type=int, default=None, help="untimed steps (default 20; 3 for c3/c5)")
    ap.add_argument("--seed", type=int, default=2024)
    ap.add_argument("--workload", default="c4",
                    choices=["c4", "c4s", "c4f", "c4g", "c2", "c3", "c3b", "c5", "ops", "readout", "matmul"])
    ap.add_argument("--kernels", default="rtc", choices=["aot", "rtc"],
                    help="how the sampler kernels are loaded: hiprtc at first use, the reference's NVRTC route "
                         "(the default; compiled by the first, untimed launch, or read from the disk cache), "
                         "or the library's hipcc code objects")
    ap.add_argument("--clock-warmup", type=float, default=1.0,
                    help="seconds of untimed launches before the warmup steps (the device's clocks settle)")
    ap.add_argument("--cpu-rows", type=int, default=256, help="rows of the CPU baseline sample (0 = skip)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="repeat the CPU sample up to this long")
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="instead of the benchmark: 20 plain device copies of this many bytes (calibrates the "
                         "FETCH_SIZE / WRITE_SIZE counters against known traffic)")
    args = ap.parse_args()
    if args.copy_bytes > 0:
        import torch
        src = torch.ones(args.copy_bytes // 4, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": src.numel() * 4, "launches": 20}), flush=True)
        return
    if args.gpus != 1:
        print(json.dumps({"error": f"--gpus {args.gpus}: this build measures one GPU; the path shards by rows "
                                   "with no exchange, and multi-GPU runs are not part of it"}))
        sys.exit(2)
    big = args.workload in ("c3", "c3b", "c5")
    if args.steps is None:
        args.steps = 20 if big else 200
    if args.warmup is None:
        args.warmup = 3 if big else 20

    import noetic_rl as nr
    import workloads as W

    if args.workload == "readout":
        # torch's own HIP runtime must find the device before the library claims it
        import torch
        torch.zeros(1, device="cuda:0")
    nr.set_kernel_path(args.kernels)
    nr.claim(0)
    if args.workload in ("c4", "c4s", "c4f", "c2"):
        out = bench_sample(nr, W, args, args.workload)
    elif args.workload == "c4g":
        out = bench_gumbel(nr, W, args)
    elif args.workload == "c3b":
        out = bench_score_grad(nr, W, args)
    elif args.workload == "ops":
        out = bench_ops(nr, args)
    elif args.workload == "matmul":
        out = bench_matmul(nr, args)
    elif args.workload == "readout":
        out = bench_readout(nr, W, args)
    else:
        out = bench_score(nr, W, args, args.workload)
    out["kernels"] = nr.kernel_path()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
