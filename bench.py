#!/usr/bin/env python3
"""bench.py -- quantized GEMV / MMQ throughput on one MI355X.

Headline workload: one decode FFN step at batch 1
through the Exec mirror (the slots the engine calls): matvecPair over the Q4_K
gate/up weights [9728,2560] x2 (adjacent in the weight arena: one launch) from
f32 x[2560], then matvec over the Q6_K down weight [2560,9728] from f32
h[9728].  The mirror quantizes x (Q8_K) inside the gate/up GEMV (one launch)
and h inside the down GEMV, split over K: each workgroup quantizes and
multiplies one 1024-value slice of h, the last one of a row tile to finish
adds the partial sums (one launch).
`value` = algorithmic bytes of the step's GEMVs (packed weights + f32 x + f32 y
per GEMV) / step time, inputs resident in HBM.  Weight sets rotate over enough
device copies (> 512 MB per pass) that every step streams from HBM, not from
the 256 MB Infinity Cache.

Also reported: the other configurations' GEMV bandwidth, the dominant
kernel's roofline fraction (HIP events around back-to-back launches of that
kernel alone), and the reference's CPU path timed on this host's cores.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1]
       python bench.py --profile-kernel down --steps 200   (one kernel only, for rocprofv3)
       python bench.py --copy-calib       (a plain copy of known size, for counter scaling)
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0     # MI355X HBM3E, vendor figure
INT8_PEAK_TOPS = 5000.0   # MI355X dense int8 MFMA (POP/s x 1e3)
ROTATE_BYTES = 512 << 20  # per-pass footprint that defeats the MALL
METRIC = "quant GEMV GB/s (% of HBM peak) at bs=1; MMQ prefill tokens/s"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gemv_bytes(rows: int, cols: int, wbytes: int, tokens: int = 1) -> int:
    """Algorithmic bytes of one GEMV: packed weights + f32 x + f32 y."""
    return wbytes + 4 * cols * tokens + 4 * rows * tokens


class Stream:
    """Device copies of a weight set, rotated per launch."""

    def __init__(self, torch, host_bytes, dev, min_bytes=ROTATE_BYTES, align=256):
        import numpy as np
        n = len(host_bytes)
        stride = (n + align - 1) // align * align
        self.copies = max(1, -(-min_bytes // stride)) if min_bytes else 1
        self.buf = torch.empty(self.copies * stride, dtype=torch.uint8, device=dev)
        src = torch.from_numpy(np.ascontiguousarray(host_bytes)).to(dev)
        for c in range(self.copies):
            self.buf[c * stride:c * stride + n].copy_(src)
        self.stride = stride
        self.n = n

    def ptr(self, i: int) -> int:
        return self.buf.data_ptr() + (i % self.copies) * self.stride


WARM_SECONDS = 0.1  # GPU clocks ramp down while the host prepares inputs


def time_loop(torch, fn, iters: int, warmup: int) -> float:
    """Average seconds per call of fn(i), HIP events on the current stream.

    Warm-up is at least `warmup` calls and at least WARM_SECONDS of back-to-back
    calls: after host-side setup the GPU's clocks have dropped, and the first
    ~10 ms of launches run measurably slower (a 357 MB GEMV read 81 us cold
    against 72 us warm on MI355X)."""
    t0 = time.perf_counter()
    i = 0
    while i < warmup or time.perf_counter() - t0 < WARM_SECONDS:
        fn(i)
        i += 1
        if i % 64 == 0:
            torch.cuda.synchronize()
    warmup = i
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(iters):
        fn(warmup + i)
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e-3 / iters


def single_latency(torch, fn, reps: int = 20) -> float:
    """Median seconds of one isolated launch (synchronized before and after)."""
    ts = []
    for i in range(reps):
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fn(i)
        b.record()
        torch.cuda.synchronize()
        ts.append(a.elapsed_time(b) * 1e-3)
    return statistics.median(ts)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="only the headline workload")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--profile-kernel", choices=["down", "gate_up", "fused_gate_up", "split_down", "step",
                                                 "step_unfused",
                                                 "mmq_cfg5_q4k", "mmq_cfg5_q3k", "mmq_cfg5_q2k",
                                                 "mmq_cfg4"],
                    help="run only this kernel (for rocprofv3) and exit")
    ap.add_argument("--copy-calib", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the quantized matvec path has no "
              "multi-GPU component; it would shard by output rows). Run with --gpus 1.",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import qwen35_amd
    from qwen35_amd import _lib, ops, synth

    lib = _lib.load()
    qwen35_amd.check("qhip_init", lib.qhip_init(0))
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream().cuda_stream
    TQ4, TQ6, TQ8, TIQ = 12, 14, 8, 20

    if args.copy_calib:
        n = 256 << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calib_bytes_read": n, "copy_calib_bytes_written": n, "launches": 5}))
        return 0

    # ---- headline workload: cfg2 FFN step through the Exec mirror --------------
    # matvecPair(gate, up, x) + matvec(down, h) (src/backend.zig:153-176 slots):
    # the mirror quantizes x and h on the device and runs one GEMV per slot
    # (adjacent gate/up weights are one launch): x inside the gate/up GEMV
    # (width 2560), h inside the split-K down launch (width 9728).
    import ctypes
    H, F = 2560, 9728
    t0 = time.time()
    wg = synth.make_weight(TQ4, F, H, seed=0, tag=1)
    wu = synth.make_weight(TQ4, F, H, seed=0, tag=2)
    wd = synth.make_weight(TQ6, H, F, seed=0, tag=3)
    x = synth.make_act(H, 1, seed=0, tag=100)
    hvec = synth.make_act(F, 1, seed=0, tag=101)
    gu_bytes, d_bytes = wg.nbytes + wu.nbytes, wd.nbytes
    set_bytes = gu_bytes + d_bytes
    copies = max(1, -(-ROTATE_BYTES // set_bytes))
    be = ops.Backend(0)
    lins = []
    for _ in range(copies):
        lg = be.load_linear(TQ4, F, H, wg)
        lu = be.load_linear(TQ4, F, H, wu)
        ld = be.load_linear(TQ6, H, F, wd)
        assert lu.dev == lg.dev + F * lg.row_bytes  # adjacent: matvecPair is one launch
        lins.append((ctypes.byref(lg), ctypes.byref(lu), ctypes.byref(ld), lg))
    sha = synth.sha256(np.concatenate([wg.reshape(-1), wu.reshape(-1), wd.reshape(-1)]))
    log(f"cfg2 weights {set_bytes / 1e6:.1f} MB x {copies} copies in the backend arena "
        f"(gen+upload {time.time() - t0:.1f}s), sha256 {sha[:16]}")
    xd = torch.from_numpy(x[0]).to(dev)
    hd = torch.from_numpy(hvec[0]).to(dev)
    y_gu = torch.empty(2 * F, device=dev)
    y_d = torch.empty(H, device=dev)
    bh = be._h
    p_x, p_h, p_ygu, p_yd = (ctypes.c_void_p(t.data_ptr()) for t in (xd, hd, y_gu, y_d))

    def gate_up(i):
        g_, u_, _, _ = lins[i % copies]
        rc = lib.qhip_backend_matvec_pair(bh, p_ygu, g_, u_, p_x)
        assert rc == 0, rc

    def down(i):
        rc = lib.qhip_backend_matvec(bh, p_yd, lins[i % copies][2], p_h)
        assert rc == 0, rc

    def step(i):
        gate_up(i)
        down(i)

    # the same step on the C ABI's separate quantize + matvec launches (4 launches)
    xq = torch.empty(lib.qhip_act_row_bytes(TQ4, H), dtype=torch.uint8, device=dev)
    hq = torch.empty(lib.qhip_act_row_bytes(TQ6, F), dtype=torch.uint8, device=dev)

    # the step's two GEMV kernels alone, on activations quantized beforehand
    assert lib.qhip_launch_quantize_act(TQ4, xd.data_ptr(), xq.data_ptr(), H, 1, stream) == 0
    assert lib.qhip_launch_quantize_act(TQ6, hd.data_ptr(), hq.data_ptr(), F, 1, stream) == 0

    def gemv_gate_up(i):
        rc = lib.qhip_launch_mul_mat_vec(lins[i % copies][3].dev, xq.data_ptr(), y_gu.data_ptr(), 2 * F, H, 1, TQ4,
                                         stream)
        assert rc == 0, rc

    def gemv_down(i):
        rc = lib.qhip_launch_mul_mat_vec(lins[i % copies][3].dev + gu_bytes, hq.data_ptr(), y_d.data_ptr(), H, F, 1,
                                         TQ6, stream)
        assert rc == 0, rc

    # the launches the mirror issues in the step: quantize + GEMV in one launch
    # for gate/up (width 2560) and, split over K, for down (9728)
    skwork = ops.split_work(H, F, dev)

    def split_down(i):
        rc = lib.qhip_launch_quantize_mul_mat_vec_split(lins[i % copies][3].dev + gu_bytes, hd.data_ptr(), None,
                                                        y_d.data_ptr(), H, F, TQ6, 0, 0, 0, skwork.data_ptr(),
                                                        skwork.numel(), stream)
        assert rc == 0, rc

    def fused_gate_up(i):
        rc = lib.qhip_launch_quantize_mul_mat_vec(lins[i % copies][3].dev, xd.data_ptr(), None, y_gu.data_ptr(),
                                                  2 * F, H, TQ4, stream)
        assert rc == 0, rc

    def quantize_h(i):
        assert lib.qhip_launch_quantize_act(TQ6, hd.data_ptr(), hq.data_ptr(), F, 1, stream) == 0

    def step_unfused(i):
        lg = lins[i % copies][3]
        assert lib.qhip_launch_quantize_act(TQ4, xd.data_ptr(), xq.data_ptr(), H, 1, stream) == 0
        assert lib.qhip_launch_mul_mat_vec(lg.dev, xq.data_ptr(), y_gu.data_ptr(), 2 * F, H, 1, TQ4, stream) == 0
        assert lib.qhip_launch_quantize_act(TQ6, hd.data_ptr(), hq.data_ptr(), F, 1, stream) == 0
        assert lib.qhip_launch_mul_mat_vec(lg.dev + gu_bytes, hq.data_ptr(), y_d.data_ptr(), H, F, 1, TQ6,
                                           stream) == 0

    if args.profile_kernel in ("down", "gate_up", "fused_gate_up", "split_down", "step", "step_unfused"):
        for i in range(3):
            step(i)
        fn = {"down": gemv_down, "gate_up": gemv_gate_up, "fused_gate_up": fused_gate_up,
              "split_down": split_down, "step": step,
              "step_unfused": step_unfused}[args.profile_kernel]
        for i in range(args.steps):
            fn(i)
        torch.cuda.synchronize()
        print(json.dumps({"profiled": args.profile_kernel, "launches": args.steps, "copies": copies}))
        return 0
    if args.profile_kernel:
        profile_mmq(torch, lib, ops, synth, dev, stream, args.profile_kernel, args.steps)
        return 0

    step_bytes = gemv_bytes(2 * F, H, gu_bytes) + gemv_bytes(H, F, d_bytes)
    sec = time_loop(torch, step, args.steps, args.warmup)
    value = step_bytes / sec / 1e9
    log(f"cfg2 step: {sec * 1e6:.2f} us, {value:.1f} GB/s ({100 * value / HBM_PEAK_GBS:.1f}% HBM)")
    sec_unfused = time_loop(torch, step_unfused, args.steps, args.warmup)
    log(f"cfg2 step, separate quantize launches: {sec_unfused * 1e6:.2f} us")

    # each launch of the step alone, back to back; the roofline's kernel is the
    # longest of them.  The GEMVs on pre-quantized activations are reported too.
    n_k = max(200, args.steps)
    gu_alg = gemv_bytes(2 * F, H, gu_bytes)
    d_alg = gemv_bytes(H, F, d_bytes)
    q_alg = 4 * F + lib.qhip_act_row_bytes(TQ6, F)
    fgu_sec = time_loop(torch, fused_gate_up, n_k, 20)
    sd_sec = time_loop(torch, split_down, n_k, 20)
    d_sec = time_loop(torch, gemv_down, n_k, 20)
    qh_sec = time_loop(torch, quantize_h, n_k, 20)
    gu_sec = time_loop(torch, gemv_gate_up, n_k, 20)

    def entry(alg, sec):
        return {"alg_bytes": alg, "avg_us": sec * 1e6, "gbs": alg / sec / 1e9}

    kernels = {
        "fused_q4_k_gate_up_19456x2560": entry(gu_alg, fgu_sec),
        "split_q6_k_down_2560x9728": entry(d_alg, sd_sec),
    }
    # the separate launches the split-K down replaces, and the gate/up GEMV on
    # a pre-quantized activation
    off_step = {"gemv_q4_k_gate_up_19456x2560_prequantized": entry(gu_alg, gu_sec),
                "gemv_q6_k_down_2560x9728_prequantized": entry(d_alg, d_sec),
                "quantize_q8_k_9728": entry(q_alg, qh_sec)}
    dom = max(kernels, key=lambda k: kernels[k]["avg_us"])
    achieved = kernels[dom]["gbs"]
    traffic = None
    tpath = ROOT / "profiles" / "traffic.json"
    if tpath.exists():
        try:
            traffic = json.loads(tpath.read_text()).get(dom, {}).get("hbm_bytes_per_launch")
        except (ValueError, AttributeError):
            traffic = None
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": dom,
                "alg_bytes_per_launch": kernels[dom]["alg_bytes"],
                "avg_launch_us": round(kernels[dom]["avg_us"], 3)}
    latency = {"gate_up_single_launch_us": round(single_latency(torch, fused_gate_up) * 1e6, 2),
               "down_single_launch_us": round(single_latency(torch, split_down) * 1e6, 2),
               "step_single_us": round(single_latency(torch, step) * 1e6, 2)}

    # ---- other configurations (GEMV bandwidth per launch, back-to-back) ------
    extra = {}
    if not args.no_extra:
        for name, tt, rows, cols in (("cfg1_q8_0_6144x1024", TQ8, 6144, 1024),
                                     ("cfg3_iq4_nl_248320x2560", TIQ, 248320, 2560),
                                     ("cfg5_q4_k_17408x5120", TQ4, 17408, 5120),
                                     ("cfg5_q6_k_5120x17408", TQ6, 5120, 17408),
                                     # further formats at the config-5 gate/up shape
                                     ("q5_k_17408x5120", 13, 17408, 5120),
                                     ("q3_k_17408x5120", 11, 17408, 5120),
                                     ("q2_k_17408x5120", 10, 17408, 5120),
                                     ("iq4_xs_17408x5120", 23, 17408, 5120),
                                     ("q4_0_17408x5120", 2, 17408, 5120),
                                     ("q4_1_17408x5120", 3, 17408, 5120),
                                     ("iq3_xxs_17408x5120", 18, 17408, 5120),
                                     ("iq3_s_17408x5120", 21, 17408, 5120)):
            t1 = time.time()
            w = synth.make_weight(tt, rows, cols, seed=0, tag=tt)
            st = Stream(torch, w.reshape(-1), dev)
            del w
            xv = torch.from_numpy(synth.make_act(cols, 1, seed=0)).to(dev)
            aq = ops.quantize_act(tt, xv)
            yo = torch.empty(rows, device=dev)

            def one(i, st=st, tt=tt, rows=rows, cols=cols, aq=aq, yo=yo):
                rc = lib.qhip_launch_mul_mat_vec(st.ptr(i), aq.data_ptr(), yo.data_ptr(), rows, cols, 1,
                                                 tt, stream)
                assert rc == 0, rc

            s = time_loop(torch, one, max(50, min(2000, int(2e9 // st.n))), 10)
            alg = gemv_bytes(rows, cols, st.n)
            extra[name] = {"gbs": round(alg / s / 1e9, 1), "hbm_frac": round(alg / s / 1e9 / HBM_PEAK_GBS, 4),
                           "avg_us": round(s * 1e6, 3), "alg_bytes": alg, "copies": st.copies,
                           "single_launch_us": round(single_latency(torch, one) * 1e6, 2)}
            log(f"{name}: {extra[name]['gbs']} GB/s, {extra[name]['avg_us']} us/launch "
                f"({st.copies} copies, {time.time() - t1:.1f}s)")
            del st
            torch.cuda.empty_cache()

    # ---- MMQ prefill: config 4 (ragged + dense 512) and config 5 crossover ------
    mmq = None
    if not args.no_extra:
        mmq = bench_mmq(torch, np, lib, ops, synth, dev, stream)

    # ---- CPU baseline: the reference's own kernels on this host ---------------
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(np, synth, wg, wu, wd, x, hvec, step_bytes, args.cpu_seconds)

    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(sec * 1e3, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (SplitMix64 seed 0, BASELINE.json config rules)",
        "config": {"workload": "cfg2 decode FFN step, batch 1, through the Exec mirror: matvecPair "
                               "Q4_K gate/up [9728,2560]x2 from f32 x[2560] + matvec Q6_K down [2560,9728] "
                               "from f32 h[9728] (Q8_K quantization on the device: of x inside the gate/up "
                               "GEMV launch, of h inside the split-K down GEMV launch)",
                   "hbm_frac": round(value / HBM_PEAK_GBS, 4), "step_alg_bytes": step_bytes,
                   "weight_copies_rotated": copies, "parallelism": "single GPU",
                   "us_per_step_separate_quantize_launches": round(sec_unfused * 1e6, 2)},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernels": kernels,
        "kernels_off_step": off_step,
        "latency": latency,
        "configs": extra,
        "mmq": mmq,
    }
    print(json.dumps(out), flush=True)
    return 0


def profile_mmq(torch, lib, ops, synth, dev, stream, which, launches):
    """Only the MMQ kernel of one configuration, for rocprofv3."""
    tt, rows, cols, T = {"mmq_cfg5_q4k": (12, 17408, 5120, 512), "mmq_cfg5_q3k": (11, 17408, 5120, 512),
                         "mmq_cfg5_q2k": (10, 17408, 5120, 512)}.get(which, (8, 3584, 1024, 512))
    w = torch.from_numpy(synth.make_weight(tt, rows, cols, seed=0, tag=tt)).to(dev)
    aq = ops.quantize_act(tt, torch.from_numpy(synth.make_act(cols, T, seed=0, tag=500 + T)).to(dev))
    y = torch.empty((T, rows), device=dev)
    for _ in range(launches):
        assert lib.qhip_launch_mul_mat(w.data_ptr(), aq.data_ptr(), y.data_ptr(), rows, cols, T, tt, 2, stream) == 0
    torch.cuda.synchronize()
    print(json.dumps({"profiled": which, "launches": launches}))


def bench_mmq(torch, np, lib, ops, synth, dev, stream):
    """Config 4: Q8_0 [3584,1024] with eight ragged sequences (lengths uniform on
    [16,256], packed by the ragged quantizer, one launch) and a dense 512-token
    sequence.  Config 5: Q4_K gate [17408,5120] and Q6_K down [5120,17408] at
    T = 1, 4, 16, 64, 512 on the GEMV and on the MMQ, and the crossover.
    Throughput: tokens/s, and 2*rows*cols*T / time against the int8 MFMA peak.
    `mmq_us` is the faster of the tile MMQ and (Q6_K) the image MMQ."""
    PATH_GEMV, PATH_MMQ = 1, 2
    res = {}

    def timed(fn, iters):
        return time_loop(torch, lambda i: fn(), iters, 3)

    def frac(rows, cols, T, sec):
        tops = 2.0 * rows * cols * T / sec / 1e12
        return round(tops, 1), round(tops / INT8_PEAK_TOPS, 4)

    # config 4
    tt, rows, cols = 8, 3584, 1024
    w = torch.from_numpy(synth.make_weight(tt, rows, cols, seed=0, tag=tt)).to(dev)
    lens = [int(v) for v in synth.ragged_lengths(8, 16, 256, seed=0)]
    seqs = [torch.from_numpy(synth.make_act(cols, n, seed=0, tag=300 + i)).to(dev) for i, n in enumerate(lens)]
    total = sum(lens)
    xq, off_d, _ = ops.quantize_ragged(tt, seqs, cols)
    ptrs = torch.tensor([q.data_ptr() for q in seqs], dtype=torch.int64, device=dev)
    yo = torch.empty((total, rows), device=dev)

    def ragged_step():
        assert lib.qhip_launch_quantize_ragged(tt, ptrs.data_ptr(), off_d.data_ptr(), len(lens), total, cols,
                                               xq.data_ptr(), stream) == 0
        assert lib.qhip_launch_mul_mat_ragged(w.data_ptr(), xq.data_ptr(), yo.data_ptr(), rows, cols,
                                              off_d.data_ptr(), len(lens), total, tt, stream) == 0

    def ragged_mmq_only():
        assert lib.qhip_launch_mul_mat_ragged(w.data_ptr(), xq.data_ptr(), yo.data_ptr(), rows, cols,
                                              off_d.data_ptr(), len(lens), total, tt, stream) == 0

    s_step = timed(ragged_step, 200)
    s_mm = timed(ragged_mmq_only, 200)
    tops, fr = frac(rows, cols, total, s_mm)
    res["cfg4_ragged_q8_0_3584x1024"] = {
        "lengths": lens, "tokens": total, "tokens_per_s": round(total / s_step, 1),
        "us_pack_quantize_and_mmq": round(s_step * 1e6, 2), "us_mmq": round(s_mm * 1e6, 2),
        "int8_tops": tops, "int8_mfma_frac": fr}
    T = 512
    xd = torch.from_numpy(synth.make_act(cols, T, seed=0, tag=400)).to(dev)
    xq5 = ops.quantize_act(tt, xd)
    y5 = torch.empty((T, rows), device=dev)
    s_d = timed(lambda: lib.qhip_launch_mul_mat(w.data_ptr(), xq5.data_ptr(), y5.data_ptr(), rows, cols, T, tt,
                                                PATH_MMQ, stream), 200)
    tops, fr = frac(rows, cols, T, s_d)
    res["cfg4_dense512_q8_0_3584x1024"] = {"tokens": T, "tokens_per_s": round(T / s_d, 1),
                                           "us_mmq": round(s_d * 1e6, 2), "int8_tops": tops, "int8_mfma_frac": fr}
    log(f"mmq cfg4: ragged {total} tokens {s_mm * 1e6:.1f} us ({res['cfg4_ragged_q8_0_3584x1024']['int8_mfma_frac']:.3f} "
        f"of int8 peak); dense 512 {s_d * 1e6:.1f} us")
    del w, xq, yo, seqs

    # config 5 sweep
    sweep = {}
    for name, tt, rows, cols in (("q4_k_17408x5120", 12, 17408, 5120), ("q6_k_5120x17408", 14, 5120, 17408)):
        w = torch.from_numpy(synth.make_weight(tt, rows, cols, seed=0, tag=tt)).to(dev)
        # the prepared MMQ weight image the Exec mirror uses for Q6_K prefill
        img = ops.mmq_image(tt, w, rows, cols) if tt == 14 else None
        rows_out = []
        cross = None
        for T in (1, 4, 16, 64, 512):
            x = torch.from_numpy(synth.make_act(cols, T, seed=0, tag=500 + T)).to(dev)
            aq = ops.quantize_act(tt, x)
            y = torch.empty((T, rows), device=dev)
            it = 100 if T <= 64 else 30
            s_g = timed(lambda: lib.qhip_launch_mul_mat(w.data_ptr(), aq.data_ptr(), y.data_ptr(), rows, cols, T, tt,
                                                        PATH_GEMV, stream), it)
            # the split-K workspace the Exec mirror passes (small grids split K)
            work = ops.mul_mat_work(rows, cols, T, tt, dev)
            wp, wn = (work.data_ptr(), work.numel()) if work is not None else (None, 0)
            s_t = timed(lambda: lib.qhip_launch_mul_mat_work(w.data_ptr(), aq.data_ptr(), y.data_ptr(), rows, cols, T,
                                                             tt, PATH_MMQ, wp, wn, stream), it)
            pt = {"T": T, "gemv_us": round(s_g * 1e6, 2), "mmq_tile_us": round(s_t * 1e6, 2)}
            s_m = s_t
            if img is not None:
                s_i = timed(lambda: lib.qhip_launch_mul_mat_image(img.data_ptr(), aq.data_ptr(), y.data_ptr(), rows,
                                                                  cols, T, tt, 0, 0, wp, wn, stream), it)
                pt["mmq_image_us"] = round(s_i * 1e6, 2)
                s_m = min(s_t, s_i)
            tops, fr = frac(rows, cols, T, s_m)
            pt.update({"mmq_us": round(s_m * 1e6, 2), "gemv_tokens_per_s": round(T / s_g, 1),
                       "mmq_tokens_per_s": round(T / s_m, 1), "mmq_int8_tops": tops, "mmq_int8_mfma_frac": fr})
            rows_out.append(pt)
            if cross is None and s_m < s_g:
                cross = T
        sweep[name] = {"points": rows_out, "crossover_T": cross}
        log(f"mmq cfg5 {name}: " + ", ".join(f"T={p['T']} gemv {p['gemv_us']} / mmq {p['mmq_us']} us"
                                              for p in rows_out) + f"; crossover T={cross}")
        del w, img
        torch.cuda.empty_cache()
    res["cfg5_sweep"] = sweep
    return res


def cpu_baseline(np, synth, wg, wu, wd, x, hvec, step_bytes, budget_s):
    """The reference's x86 kernels (oracle/_ref, compiled from its sources) on
    this host's cores: Q8_K quantize + row dots with the reference pool's chunk
    rule, rotating weight copies (>512 MB) like the GPU does."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import pyoracle
    orc = pyoracle.Oracle()
    ref = pyoracle.load_ref()
    kind = "reference" if ref is not None else "port"
    threads = pyoracle.host_threads()
    H, F = x.shape[1], hvec.shape[1]
    gu = np.concatenate([wg, wu])
    one = gu.nbytes + wd.nbytes
    copies = max(1, -(-ROTATE_BYTES // one))
    gus = [gu.copy() for _ in range(copies)]
    wds = [wd.copy() for _ in range(copies)]
    quant = (ref or orc).quantize_act
    dot4 = ref.dot_fn_addr(12) if ref else orc.dot_fn_addr(12)
    dot6 = ref.dot_fn_addr(14) if ref else orc.dot_fn_addr(14)
    y1 = np.empty((1, 2 * F), np.float32)
    y2 = np.empty((1, H), np.float32)

    def step(i, nt):
        xq = quant(12, x)
        orc.matvec_q_fn(dot4, 12, gus[i % copies], xq, H, y1, nt)
        hq = quant(14, hvec)
        orc.matvec_q_fn(dot6, 14, wds[i % copies], hq, F, y2, nt)

    res = {}
    for nt in (threads, 1):
        for i in range(2):
            step(i, nt)
        ts, i = [], 0
        deadline = time.time() + (budget_s if nt == threads else budget_s / 3)
        while len(ts) < 200:
            t = time.perf_counter()
            step(i, nt)
            ts.append(time.perf_counter() - t)
            i += 1
            if len(ts) >= 5 and time.time() > deadline:
                break
        res[nt] = (statistics.median(ts), len(ts))
    med, n = res[threads]
    tier = ref.tier() if ref else "scalar port"
    log(f"cpu baseline ({kind}, {threads} threads, {tier}): {med * 1e3:.2f} ms/step, "
        f"{step_bytes / med / 1e9:.2f} GB/s; 1 thread {res[1][0] * 1e3:.2f} ms")
    return {"value": round(step_bytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": kind,
            "sample": f"cfg2 FFN step (Q8_K quantize + Q4_K 2x[9728,2560] + Q6_K [2560,9728] row dots), "
                      f"median of {n} steps over {copies} rotating weight copies, tier {tier}",
            "ms_per_step": round(med * 1e3, 3),
            "one_thread_gbs": round(step_bytes / res[1][0] / 1e9, 3)}


if __name__ == "__main__":
    sys.exit(main())
