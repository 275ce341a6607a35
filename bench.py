#!/usr/bin/env python3
"""bench.py -- quantized GEMV / MMQ throughput on one MI355X.

Headline (BASELINE.json metric "quant GEMV GB/s (% of HBM peak) at bs=1", on
its largest single-GPU configuration, configs[2]): the IQ4_NL output-head
GEMV [248320, 2560] at batch 1, as the engine calls it -- the Exec mirror's
matvec from f32 x (Q8_0 quantization of x on the device, then the GEMV).  The
357 MB weight is larger than the 256 MB Infinity Cache, so every launch
streams it from HBM.  The Exec mirror keeps the weight's GEMV image (the same
bytes per row, quant bytes 16-byte aligned in the order the kernel walks
them), built at load time, and multiplies from it.  `value` = algorithmic bytes (packed weights + f32 x +
f32 y = 358,584,320 B) / step time, inputs resident in HBM.  `roofline` is the
GEMV kernel alone (the step's dominant kernel), timed with HIP events on its
launch stream.

Also reported: the config-2 decode FFN step (gate/up + down through the Exec
mirror) and its kernels, the GEMV bandwidth of configs 1 and 5 and of the
further formats, the MMQ (config 4 ragged and dense, the config-5 token sweep
and its GEMV->MMQ crossover), and the CPU baseline: this repository's C
restatement of the reference's CPU path at the host's ISA tier (oracle/,
AVX2 / AVX-512 VNNI as the reference dispatches them) on every configuration.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1]
       python bench.py --profile-kernel cfg3_gemv --steps 200   (one kernel only, for rocprofv3)
       python bench.py --copy-calib       (a plain copy of known size, for counter scaling)
"""
from __future__ import annotations

import argparse
import ctypes
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
TQ8, TQ4, TQ6, TIQ = 8, 12, 14, 20
PATH_AUTO, PATH_GEMV, PATH_MMQ = 0, 1, 2
H2, F2 = 2560, 9728          # config 2 (4B-class FFN)
R3, C3 = 248320, 2560        # config 3 (output head)

PROFILE_KERNELS = ["cfg3_gemv", "cfg3_step", "cfg3_gemv_gguf", "cfg1_gemv", "cfg5_q4k_gemv", "cfg5_q6k_gemv",
                   "cfg5_q6k_kimage",
                   "down", "gate_up", "fused_gate_up", "split_down", "mirror_down", "step", "step_unfused",
                   "mmq_cfg4", "mmq_cfg5_q4k", "mmq_cfg5_q6k_image", "mmq_cfg5_q3k", "mmq_cfg5_q2k",
                   "mmq_cfg5_q4k_frag", "mmq_cfg5_q4k_frag_t8", "mmq_cfg5_q6k_frag_t8", "mmq_cfg5_q6k_frag_t64",
                   "mmq_cfg4_frag",
                   "mmq_cfg4_ragged_frag"]


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
    """Average seconds per call of fn(i), HIP events on the current stream (the
    stream every launch here goes to).

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


def traffic_for(kernel: str):
    """HBM bytes per launch of `kernel` from the committed counter summary
    (FETCH_SIZE and WRITE_SIZE, scaled by a plain copy's readings)."""
    tpath = ROOT / "profiles" / "traffic.json"
    try:
        return json.loads(tpath.read_text()).get(kernel, {}).get("hbm_bytes_per_launch")
    except (OSError, ValueError, AttributeError):
        return None


class Ctx:
    def __init__(self, torch, np, lib, ops, synth, dev, stream):
        self.torch, self.np, self.lib, self.ops, self.synth = torch, np, lib, ops, synth
        self.dev, self.stream = dev, stream


# ---- config 3: the headline ------------------------------------------------------------

class Cfg3:
    """The IQ4_NL output head through the Exec mirror (resident weight, its
    GEMV image built at load time) and its GEMV kernel alone on a
    pre-quantized activation: the image GEMV the step runs, and the
    GGUF-layout GEMV for comparison."""

    def __init__(self, c: Ctx):
        self.c = c
        torch, ops, synth, lib = c.torch, c.ops, c.synth, c.lib
        t0 = time.time()
        w = synth.make_weight(TIQ, R3, C3, seed=0, tag=TIQ)
        self.x = synth.make_act(C3, 1, seed=0, tag=103)
        self.sha = synth.sha256(w)
        self.be = ops.Backend(0)
        self.lin = self.be.load_linear(TIQ, R3, C3, w)
        assert self.be.prepare_linear(self.lin) == 0  # the GEMV image
        self.wbytes = w.nbytes
        self.w_host = w
        self.xd = torch.from_numpy(self.x[0]).to(c.dev)
        self.y = torch.empty(R3, device=c.dev)
        self.xq = ops.quantize_act(TIQ, self.xd)
        # the kernels alone: a second copy of the weight and its image
        wd = torch.from_numpy(w).to(c.dev)
        self.img = ops.gemv_image(TIQ, wd, R3, C3)
        del wd
        self.xa = ops.quantize_act_image(TIQ, self.xd)
        self.alg = gemv_bytes(R3, C3, self.wbytes)
        self._p = [ctypes.c_void_p(t.data_ptr()) for t in (self.y, self.xd)]
        self._lin = ctypes.byref(self.lin)
        log(f"cfg3 IQ4_NL [{R3}x{C3}] {self.wbytes / 1e6:.1f} MB resident (gen+upload {time.time() - t0:.1f}s), "
            f"sha256 {self.sha[:16]}")

    def step(self, i=0):
        rc = self.c.lib.qhip_backend_matvec(self.be._h, self._p[0], self._lin, self._p[1])
        assert rc == 0, rc

    def gemv(self, i=0):
        rc = self.c.lib.qhip_launch_mul_mat_vec_image(self.img.data_ptr(), self.xa.data_ptr(), self.y.data_ptr(),
                                                      R3, C3, TIQ, 0, self.c.stream)
        assert rc == 0, rc

    def gemv_gguf(self, i=0):
        rc = self.c.lib.qhip_launch_mul_mat_vec(self.lin.dev, self.xq.data_ptr(), self.y.data_ptr(), R3, C3, 1, TIQ,
                                                self.c.stream)
        assert rc == 0, rc

    def quantize(self, i=0):
        rc = self.c.lib.qhip_launch_quantize_act_image(TIQ, self.xd.data_ptr(), self.xa.data_ptr(), C3, 1,
                                                       self.c.stream)
        assert rc == 0, rc


# ---- config 2: decode FFN step through the Exec mirror ----------------------------------

class Cfg2:
    """matvecPair(gate, up, x) + matvec(down, h) (src/backend.zig:153-176 slots):
    the mirror quantizes x and h on the device and runs one launch per slot --
    x inside the fused gate/up GEMV (width 2560), h inside the split-K down GEMV
    (width 9728).  Weight sets rotate over enough copies (> 512 MB per pass)
    that every step streams from HBM."""

    def __init__(self, c: Ctx):
        self.c = c
        torch, np, ops, synth, lib = c.torch, c.np, c.ops, c.synth, c.lib
        t0 = time.time()
        self.wg = synth.make_weight(TQ4, F2, H2, seed=0, tag=1)
        self.wu = synth.make_weight(TQ4, F2, H2, seed=0, tag=2)
        self.wd = synth.make_weight(TQ6, H2, F2, seed=0, tag=3)
        self.x = synth.make_act(H2, 1, seed=0, tag=100)
        self.h = synth.make_act(F2, 1, seed=0, tag=101)
        self.gu_bytes, self.d_bytes = self.wg.nbytes + self.wu.nbytes, self.wd.nbytes
        set_bytes = self.gu_bytes + self.d_bytes
        self.copies = max(1, -(-ROTATE_BYTES // set_bytes))
        self.be = ops.Backend(0)
        self.lins = []
        for _ in range(self.copies):
            lg = self.be.load_linear(TQ4, F2, H2, self.wg)
            lu = self.be.load_linear(TQ4, F2, H2, self.wu)
            ld = self.be.load_linear(TQ6, H2, F2, self.wd)
            assert lu.dev == lg.dev + F2 * lg.row_bytes  # adjacent: matvecPair is one launch
            self.lins.append((ctypes.byref(lg), ctypes.byref(lu), ctypes.byref(ld), lg))
        log(f"cfg2 weights {set_bytes / 1e6:.1f} MB x {self.copies} copies in the backend arena "
            f"(gen+upload {time.time() - t0:.1f}s)")
        self.xd = torch.from_numpy(self.x[0]).to(c.dev)
        self.hd = torch.from_numpy(self.h[0]).to(c.dev)
        self.y_gu = torch.empty(2 * F2, device=c.dev)
        self.y_d = torch.empty(H2, device=c.dev)
        self._p = [ctypes.c_void_p(t.data_ptr()) for t in (self.xd, self.hd, self.y_gu, self.y_d)]
        self.xq = torch.empty(lib.qhip_act_row_bytes(TQ4, H2), dtype=torch.uint8, device=c.dev)
        self.hq = torch.empty(lib.qhip_act_row_bytes(TQ6, F2), dtype=torch.uint8, device=c.dev)
        assert lib.qhip_launch_quantize_act(TQ4, self.xd.data_ptr(), self.xq.data_ptr(), H2, 1, c.stream) == 0
        assert lib.qhip_launch_quantize_act(TQ6, self.hd.data_ptr(), self.hq.data_ptr(), F2, 1, c.stream) == 0
        self.skwork = ops.split_work(H2, F2, c.dev)
        self.step_bytes = gemv_bytes(2 * F2, H2, self.gu_bytes) + gemv_bytes(H2, F2, self.d_bytes)

    def gate_up(self, i):
        g_, u_, _, _ = self.lins[i % self.copies]
        assert self.c.lib.qhip_backend_matvec_pair(self.be._h, self._p[2], g_, u_, self._p[0]) == 0

    def down(self, i):
        assert self.c.lib.qhip_backend_matvec(self.be._h, self._p[3], self.lins[i % self.copies][2], self._p[1]) == 0

    def step(self, i):
        self.gate_up(i)
        self.down(i)

    def base(self, i):
        return self.lins[i % self.copies][3].dev

    def gemv_gate_up(self, i):
        assert self.c.lib.qhip_launch_mul_mat_vec(self.base(i), self.xq.data_ptr(), self.y_gu.data_ptr(), 2 * F2, H2,
                                                  1, TQ4, self.c.stream) == 0

    def gemv_down(self, i):
        assert self.c.lib.qhip_launch_mul_mat_vec(self.base(i) + self.gu_bytes, self.hq.data_ptr(),
                                                  self.y_d.data_ptr(), H2, F2, 1, TQ6, self.c.stream) == 0

    def split_down(self, i):
        assert self.c.lib.qhip_launch_quantize_mul_mat_vec_split(
            self.base(i) + self.gu_bytes, self.hd.data_ptr(), None, self.y_d.data_ptr(), H2, F2, TQ6, 0, 0, 0,
            self.skwork.data_ptr(), self.skwork.numel(), self.c.stream) == 0

    def fused_gate_up(self, i):
        assert self.c.lib.qhip_launch_quantize_mul_mat_vec(self.base(i), self.xd.data_ptr(), None,
                                                           self.y_gu.data_ptr(), 2 * F2, H2, TQ4, self.c.stream) == 0

    def quantize_h(self, i):
        assert self.c.lib.qhip_launch_quantize_act(TQ6, self.hd.data_ptr(), self.hq.data_ptr(), F2, 1,
                                                   self.c.stream) == 0

    def step_unfused(self, i):
        L, s = self.c.lib, self.c.stream
        assert L.qhip_launch_quantize_act(TQ4, self.xd.data_ptr(), self.xq.data_ptr(), H2, 1, s) == 0
        self.gemv_gate_up(i)
        self.quantize_h(i)
        self.gemv_down(i)

    def run(self, steps, warmup):
        torch = self.c.torch
        sec = time_loop(torch, self.step, steps, warmup)
        sec_unfused = time_loop(torch, self.step_unfused, steps, warmup)
        n_k = max(200, steps)
        gu_alg = gemv_bytes(2 * F2, H2, self.gu_bytes)
        d_alg = gemv_bytes(H2, F2, self.d_bytes)

        def entry(alg, s):
            return {"alg_bytes": alg, "avg_us": round(s * 1e6, 3), "gbs": round(alg / s / 1e9, 1),
                    "hbm_frac": round(alg / s / 1e9 / HBM_PEAK_GBS, 4)}

        res = {"workload": "matvecPair Q4_K gate/up [9728,2560]x2 from f32 x[2560] (one fused quantize + GEMV "
                           "launch) + matvec Q6_K down [2560,9728] from f32 h[9728] (quantize, then the GEMV from "
                           "the weight's K-quant image) through the Exec mirror",
               "step_alg_bytes": self.step_bytes, "us_per_step": round(sec * 1e6, 3),
               "gbs": round(self.step_bytes / sec / 1e9, 1),
               "hbm_frac": round(self.step_bytes / sec / 1e9 / HBM_PEAK_GBS, 4),
               "us_per_step_separate_quantize_launches": round(sec_unfused * 1e6, 2),
               "weight_copies_rotated": self.copies,
               "kernels": {"fused_q4_k_gate_up_19456x2560": entry(gu_alg, time_loop(torch, self.fused_gate_up, n_k, 20)),
                           # the mirror's down matvec: quantize h, then the GEMV from the K-quant image
                           "mirror_q6_k_down_2560x9728": entry(d_alg, time_loop(torch, self.down, n_k, 20))},
               "kernels_off_step": {
                   "split_q6_k_down_2560x9728": entry(d_alg, time_loop(torch, self.split_down, n_k, 20)),
                   "gemv_q4_k_gate_up_19456x2560_prequantized": entry(gu_alg, time_loop(torch, self.gemv_gate_up, n_k, 20)),
                   "gemv_q6_k_down_2560x9728_prequantized": entry(d_alg, time_loop(torch, self.gemv_down, n_k, 20)),
                   "quantize_q8_k_9728": entry(4 * F2 + self.c.lib.qhip_act_row_bytes(TQ6, F2),
                                               time_loop(torch, self.quantize_h, n_k, 20))},
               "step_single_launch_us": round(single_latency(torch, self.step) * 1e6, 2)}
        log(f"cfg2 step: {res['us_per_step']} us, {res['gbs']} GB/s ({100 * res['hbm_frac']:.1f}% HBM); "
            f"separate quantize launches {res['us_per_step_separate_quantize_launches']} us")
        return res


# ---- other GEMV configurations -----------------------------------------------------------

GEMV_CONFIGS = (("cfg1_q8_0_6144x1024", TQ8, 6144, 1024),
                ("cfg5_q4_k_17408x5120", TQ4, 17408, 5120),
                ("cfg5_q6_k_5120x17408", TQ6, 5120, 17408),
                # the benchmark formats Q8_0 and IQ4_NL, and the further
                # formats, at the config-5 gate/up shape
                ("q8_0_17408x5120", TQ8, 17408, 5120),
                ("iq4_nl_17408x5120", TIQ, 17408, 5120),
                ("q5_k_17408x5120", 13, 17408, 5120),
                ("q3_k_17408x5120", 11, 17408, 5120),
                ("q2_k_17408x5120", 10, 17408, 5120),
                ("iq4_xs_17408x5120", 23, 17408, 5120),
                ("q4_0_17408x5120", 2, 17408, 5120),
                ("q4_1_17408x5120", 3, 17408, 5120),
                ("iq3_xxs_17408x5120", 18, 17408, 5120),
                ("iq3_s_17408x5120", 21, 17408, 5120))


def gemv_stream(c: Ctx, tt, rows, cols):
    w = c.synth.make_weight(tt, rows, cols, seed=0, tag=tt)
    st = Stream(c.torch, w.reshape(-1), c.dev)
    xv = c.torch.from_numpy(c.synth.make_act(cols, 1, seed=0)).to(c.dev)
    aq = c.ops.quantize_act(tt, xv)
    yo = c.torch.empty(rows, device=c.dev)

    def one(i):
        rc = c.lib.qhip_launch_mul_mat_vec(st.ptr(i), aq.data_ptr(), yo.data_ptr(), rows, cols, 1, tt, c.stream)
        assert rc == 0, rc
    return st, one, (aq, yo)


def bench_gemv_configs(c: Ctx):
    extra = {}
    for name, tt, rows, cols in GEMV_CONFIGS:
        t1 = time.time()
        st, one, keep = gemv_stream(c, tt, rows, cols)
        iters = max(50, min(2000, int(2e9 // st.n)))
        s = time_loop(c.torch, one, iters, 10)
        alg = gemv_bytes(rows, cols, st.n)
        extra[name] = {"gbs": round(alg / s / 1e9, 1), "hbm_frac": round(alg / s / 1e9 / HBM_PEAK_GBS, 4),
                       "avg_us": round(s * 1e6, 3), "alg_bytes": alg, "copies": st.copies,
                       "single_launch_us": round(single_latency(c.torch, one) * 1e6, 2)}
        if c.lib.qhip_gemv_image_bytes(tt, rows, cols) > 0 and rows * cols > (1 << 23):
            # the formats with a GEMV weight image: what the Exec mirror reads
            # for one token (the same bytes reordered, rotated alike), on the
            # split activation
            imgs = [c.ops.gemv_image(tt, st.buf[k * st.stride:k * st.stride + st.n], rows, cols)
                    for k in range(st.copies)]
            x = c.torch.from_numpy(c.synth.make_act(cols, 1, seed=0, tag=104)).to(c.dev)
            xa = c.ops.quantize_act_image(tt, x)
            y = c.torch.empty(rows, device=c.dev)
            img_one = lambda i: c.lib.qhip_launch_mul_mat_vec_image(imgs[i % len(imgs)].data_ptr(), xa.data_ptr(),
                                                                   y.data_ptr(), rows, cols, tt, 0, c.stream)
            si = time_loop(c.torch, img_one, iters, 10)
            extra[name].update({"image_gbs": round(alg / si / 1e9, 1),
                                "image_hbm_frac": round(alg / si / 1e9 / HBM_PEAK_GBS, 4),
                                "image_avg_us": round(si * 1e6, 3)})
            del imgs
        log(f"{name}: {extra[name]['gbs']} GB/s, {extra[name]['avg_us']} us/launch "
            + (f"(GEMV image {extra[name]['image_gbs']} GB/s, {extra[name]['image_avg_us']} us) "
               if "image_gbs" in extra[name] else "")
            + f"({st.copies} copies, {time.time() - t1:.1f}s)")
        del st, keep
        c.torch.cuda.empty_cache()
    return extra


# ---- MMQ ------------------------------------------------------------------------------------

def bench_mmq(c: Ctx):
    """Config 4: Q8_0 [3584,1024] with eight ragged sequences (lengths uniform on
    [16,256], packed by the ragged quantizer, one launch) and a dense 512-token
    sequence.  Config 5: Q4_K gate [17408,5120] and Q6_K down [5120,17408] at
    T = 1, 2, 4, 8, 16, 32, 64, 512 on the GEMV and on the MMQ (with the
    split-K workspace the Exec mirror passes), and the crossover; weight
    copies (with their images) rotated per launch past the Infinity Cache.
    Throughput: tokens/s, and 2*rows*cols*T / time against the int8 MFMA
    peak.  `mmq_us`
    is the fastest of the MMQ on the GGUF rows, from the fragment image and
    (Q6_K) from the MMQ image; `mirror_us` is what the Exec mirror launches
    (Q6_K at one token: the GEMV from the K-quant image)."""
    torch, lib, ops, synth, dev, stream = c.torch, c.lib, c.ops, c.synth, c.dev, c.stream
    res = {}

    def timed(fn, iters):
        return time_loop(torch, lambda i: fn(), iters, 3)

    def frac(rows, cols, T, sec):
        tops = 2.0 * rows * cols * T / sec / 1e12
        return round(tops, 1), round(tops / INT8_PEAK_TOPS, 4)

    tt, rows, cols = TQ8, 3584, 1024
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
    mem = 3899392 + 4 * cols * T + 4 * rows * T
    res["cfg4_dense512_q8_0_3584x1024"] = {"tokens": T, "tokens_per_s": round(T / s_d, 1),
                                           "us_mmq": round(s_d * 1e6, 2), "int8_tops": tops, "int8_mfma_frac": fr,
                                           "alg_bytes": mem, "hbm_frac": round(mem / s_d / 1e9 / HBM_PEAK_GBS, 4)}
    # what the Exec mirror launches for these (K <= 1024, from 6 tokens): the
    # MMQ from the weight's Q8_0 fragment image, on the same packed rows
    img8 = ops.wd_image(tt, w, rows, cols)
    s_ri = timed(lambda: lib.qhip_launch_mul_mat_wd_image(img8.data_ptr(), xq.data_ptr(), yo.data_ptr(), rows, cols,
                                                          total, tt, None, 0, stream), 200)
    s_di = timed(lambda: lib.qhip_launch_mul_mat_wd_image(img8.data_ptr(), xq5.data_ptr(), y5.data_ptr(), rows, cols,
                                                          T, tt, None, 0, stream), 200)
    # and end to end: the f32 activations quantized (the ragged batch packed)
    # then the fragment-image MMQ
    def ragged_mirror_step():
        assert lib.qhip_launch_quantize_ragged(tt, ptrs.data_ptr(), off_d.data_ptr(), len(lens), total, cols,
                                               xq.data_ptr(), stream) == 0
        assert lib.qhip_launch_mul_mat_wd_image(img8.data_ptr(), xq.data_ptr(), yo.data_ptr(), rows, cols, total,
                                                tt, None, 0, stream) == 0

    def dense_mirror_step():
        assert lib.qhip_launch_quantize_act(tt, xd.data_ptr(), xq5.data_ptr(), cols, T, stream) == 0
        assert lib.qhip_launch_mul_mat_wd_image(img8.data_ptr(), xq5.data_ptr(), y5.data_ptr(), rows, cols, T, tt,
                                                None, 0, stream) == 0

    s_rs = timed(ragged_mirror_step, 200)
    s_ds = timed(dense_mirror_step, 200)
    for key, sec, nt, step in (("cfg4_ragged_q8_0_3584x1024", s_ri, total, s_rs),
                               ("cfg4_dense512_q8_0_3584x1024", s_di, T, s_ds)):
        tops, fr = frac(rows, cols, nt, sec)
        res[key].update({"us_mmq_fragment_image": round(sec * 1e6, 2), "fragment_image_int8_tops": tops,
                         "fragment_image_int8_mfma_frac": fr, "mirror_path": "fragment_image",
                         "mirror_us": round(sec * 1e6, 2),
                         "us_quantize_and_mirror_mmq": round(step * 1e6, 2),
                         "mirror_tokens_per_s": round(nt / step, 1)})
    log(f"mmq cfg4: ragged {total} tokens {s_mm * 1e6:.1f} us (fragment image {s_ri * 1e6:.1f}) "
        f"({res['cfg4_ragged_q8_0_3584x1024']['int8_mfma_frac']:.3f} of int8 peak); dense 512 {s_d * 1e6:.1f} us "
        f"(fragment image {s_di * 1e6:.1f})")
    del w, xq, yo, seqs, img8

    sweep = {}

    def rotated(fn, iters):
        return time_loop(torch, fn, iters, 3)

    for name, tt, rows, cols in (("q4_k_17408x5120", TQ4, 17408, 5120), ("q6_k_5120x17408", TQ6, 5120, 17408)):
        # weight copies, each with the images the Exec mirror derives from it
        # (the fragment image it reads from 2 tokens, Q6_K's MMQ image from
        # 65), rotated per launch so that every launch streams its weight
        # from HBM as a decode does (one copy would stay in the 256 MB
        # Infinity Cache)
        wh = synth.make_weight(tt, rows, cols, seed=0, tag=tt)
        ncopy = max(1, -(-ROTATE_BYTES // wh.nbytes))
        ws = [torch.from_numpy(wh).to(dev) for _ in range(ncopy)]
        frags = [ops.wd_image(tt, w, rows, cols) for w in ws]
        imgs = [ops.mmq_image(tt, w, rows, cols) for w in ws] if tt == TQ6 else None
        kimgs = [ops.gemv_image(tt, w, rows, cols) for w in ws] if tt == TQ6 else None
        rows_out = []
        cross = None
        for T in (1, 2, 4, 8, 16, 32, 64, 512):
            x = torch.from_numpy(synth.make_act(cols, T, seed=0, tag=500 + T)).to(dev)
            aq = ops.quantize_act(tt, x)
            y = torch.empty((T, rows), device=dev)
            it = 100 if T <= 64 else 30
            # the split-K workspace the Exec mirror passes (small grids split K)
            work = ops.mul_mat_work(rows, cols, T, tt, dev)
            wp, wn = (work.data_ptr(), work.numel()) if work is not None else (None, 0)
            s_g = rotated(lambda i: lib.qhip_launch_mul_mat(ws[i % ncopy].data_ptr(), aq.data_ptr(), y.data_ptr(),
                                                            rows, cols, T, tt, PATH_GEMV, stream), it)
            s_t = rotated(lambda i: lib.qhip_launch_mul_mat_work(ws[i % ncopy].data_ptr(), aq.data_ptr(),
                                                                 y.data_ptr(), rows, cols, T, tt, PATH_MMQ, wp, wn,
                                                                 stream), it)
            pt = {"T": T, "gemv_us": round(s_g * 1e6, 2), "mmq_tile_us": round(s_t * 1e6, 2)}
            s_m = s_t
            s_i = None
            if imgs is not None:
                s_i = rotated(lambda i: lib.qhip_launch_mul_mat_image(imgs[i % ncopy].data_ptr(), aq.data_ptr(),
                                                                      y.data_ptr(), rows, cols, T, tt, 0, 0, wp, wn,
                                                                      stream), it)
                pt["mmq_image_us"] = round(s_i * 1e6, 2)
                s_m = min(s_t, s_i)
            s_f = None
            if tt == TQ4 or T <= 64:
                s_f = rotated(lambda i: lib.qhip_launch_mul_mat_wd_image(frags[i % ncopy].data_ptr(), aq.data_ptr(),
                                                                         y.data_ptr(), rows, cols, T, tt, wp, wn,
                                                                         stream), it)
                pt["mmq_fragment_image_us"] = round(s_f * 1e6, 2)
                s_m = min(s_m, s_f)
            # the C ABI's automatic path (GEMV or tile MMQ by the measured
            # crossover), and what the Exec mirror's matvecBatchK launches: the
            # same, except the fragment image from 2 tokens (Q6_K up to 64)
            # and the Q6_K MMQ image from 65
            s_a = rotated(lambda i: lib.qhip_launch_mul_mat_work(ws[i % ncopy].data_ptr(), aq.data_ptr(),
                                                                 y.data_ptr(), rows, cols, T, tt, PATH_AUTO, wp, wn,
                                                                 stream), it)
            pt["auto_us"] = round(s_a * 1e6, 2)
            s_k = None
            if kimgs is not None and T == 1:
                # the GEMV from the K-quant image (the activation in the same
                # Q8_K rows)
                s_k = rotated(lambda i: lib.qhip_launch_mul_mat_vec_image(kimgs[i % ncopy].data_ptr(), aq.data_ptr(),
                                                                          y.data_ptr(), rows, cols, tt, 0, stream), it)
                pt["gemv_kimage_us"] = round(s_k * 1e6, 2)
            s_mirror = (s_i if s_i is not None and T > 64 else s_f if s_f is not None and T >= 2 else
                        s_k if s_k is not None else s_a)
            pt["mirror_path"] = ("mmq_image" if s_i is not None and T > 64 else
                                 "fragment_image" if s_f is not None and T >= 2 else
                                 "gemv_kimage" if s_k is not None else "auto")
            pt["mirror_us"] = round(s_mirror * 1e6, 2)
            if s_mirror > 1.1 * min(s_g, s_m):
                pt["mirror_warning"] = "the Exec mirror's choice is more than 10% slower than the fastest path"
                log(f"WARNING: {name} T={T}: mirror {s_mirror * 1e6:.2f} us vs GEMV {s_g * 1e6:.2f} / "
                    f"MMQ {s_m * 1e6:.2f} us")
            tops, fr = frac(rows, cols, T, s_m)
            pt.update({"mmq_us": round(s_m * 1e6, 2), "gemv_tokens_per_s": round(T / s_g, 1),
                       "mmq_tokens_per_s": round(T / s_m, 1), "mmq_int8_tops": tops, "mmq_int8_mfma_frac": fr})
            rows_out.append(pt)
            if cross is None and s_m < s_g:
                cross = T
        # small batches against one token: what the Exec mirror launches at
        # 2..8 tokens over the batch-1 GEMV on the GGUF rows, and over what
        # it launches for one token
        t1 = next(p["gemv_us"] for p in rows_out if p["T"] == 1)
        m1 = next(p["mirror_us"] for p in rows_out if p["T"] == 1)
        worst = max(p["mirror_us"] for p in rows_out if 2 <= p["T"] <= 8)
        sweep[name] = {"points": rows_out, "crossover_T": cross, "mirror_2_8_over_gemv_1": round(worst / t1, 3),
                       "mirror_2_8_over_mirror_1": round(worst / m1, 3), "weight_copies": ncopy}
        log(f"mmq cfg5 {name}: " + ", ".join(f"T={p['T']} gemv {p['gemv_us']} / mmq {p['mmq_us']} us"
                                              for p in rows_out) + f"; crossover T={cross}")
        del ws, imgs, frags, kimgs
        torch.cuda.empty_cache()
    res["cfg5_sweep"] = sweep
    return res


# ---- CPU baseline ----------------------------------------------------------------------------

def cpu_time(fn, budget_s, min_reps=5, max_reps=200):
    """Median seconds of fn() after one warm-up call, within a time budget."""
    fn(0)
    ts, i = [], 1
    deadline = time.time() + budget_s
    while len(ts) < max_reps:
        t = time.perf_counter()
        fn(i)
        ts.append(time.perf_counter() - t)
        i += 1
        if len(ts) >= min_reps and time.time() > deadline:
            break
    return statistics.median(ts), len(ts)


def cpu_baseline(c: Ctx, cfg3: Cfg3, cfg2: Cfg2 | None, budget_s: float, all_configs: bool):
    """This repository's C restatement of the reference CPU path (oracle/): the
    activation quantized once per token, then one row dot per (token, row) at
    the host's ISA tier (IQ4_NL / Q4_K / Q6_K AVX2, Q8_0 AVX-512 VNNI, as the
    reference dispatches), row-parallel with the reference pool's chunk rule
    (src/pool.zig:489-494) over the host cores this process may use."""
    np, synth = c.np, c.synth
    sys.path.insert(0, str(ROOT / "oracle"))
    import pyoracle
    orc = pyoracle.Oracle()
    threads = pyoracle.host_threads()
    nproc = os.cpu_count()

    def gemv_case(tt, W, x, rows, cols, copies=1):
        """quantize x once, then the row dots; weight copies rotated."""
        dot = orc.simd_dot_fn_addr(tt)
        Ws = [W] + [W.copy() for _ in range(copies - 1)]
        y = np.empty((x.shape[0], rows), np.float32)

        def run(i, nt):
            act = orc.quantize_act(tt, x)
            orc.matvec_q_fn(dot, tt, Ws[i % copies], act, cols, y, nt)
        return run

    res = {"kind": "port", "cores": threads, "host_nproc": nproc, "configs": {}}

    def record(name, run, alg, unit_den, budget, unit="GB/s", extra=None):
        med, n = cpu_time(lambda i: run(i, threads), budget)
        med1, n1 = cpu_time(lambda i: run(i, 1), budget / 3, min_reps=3)
        if unit == "GB/s":
            v, v1 = alg / med / 1e9, alg / med1 / 1e9
        else:
            v, v1 = unit_den / med, unit_den / med1
        ent = {"value": round(v, 3), "unit": unit, "threads": threads, "ms": round(med * 1e3, 3), "reps": n,
               "one_thread_value": round(v1, 3), "one_thread_ms": round(med1 * 1e3, 3)}
        if extra:
            ent.update(extra)
        res["configs"][name] = ent
        log(f"cpu {name}: {v:.2f} {unit} on {threads} threads ({med * 1e3:.2f} ms), 1 thread {v1:.2f}")
        return ent

    # config 3 (the headline workload), the whole GEMV
    r3 = gemv_case(TIQ, cfg3.w_host, cfg3.x, R3, C3)
    head = record("cfg3_iq4_nl_248320x2560", r3, cfg3.alg, None, budget_s * 0.4,
                  extra={"tier": orc.simd_tier(TIQ)})
    res.update({"value": head["value"], "unit": "GB/s", "tier": orc.simd_tier(TIQ),
                "sample": f"the whole config-3 GEMV (Q8_0 quantize of x[2560] + 248320 IQ4_NL row dots, AVX2 "
                          f"codebook shuffle), median of {head['reps']} runs on {threads} threads "
                          f"(host nproc {nproc}); 1 thread {head['one_thread_value']} GB/s"})
    if not all_configs:
        return res
    budget = budget_s * 0.6 / 6
    # config 1: Q8_0 [6144, 1024], copies rotated past 512 MB like the GPU
    w1 = synth.make_weight(TQ8, 6144, 1024, seed=0, tag=TQ8)
    x1 = synth.make_act(1024, 1, seed=0)
    record("cfg1_q8_0_6144x1024", gemv_case(TQ8, w1, x1, 6144, 1024, copies=max(1, ROTATE_BYTES // w1.nbytes)),
           gemv_bytes(6144, 1024, w1.nbytes), None, budget, extra={"tier": orc.simd_tier(TQ8)})
    del w1
    # config 2: the decode FFN step (quantize x, gate/up dots, quantize h, down dots)
    if cfg2 is not None:
        gu = np.concatenate([cfg2.wg, cfg2.wu])
        r_gu = gemv_case(TQ4, gu, cfg2.x, 2 * F2, H2, copies=cfg2.copies)
        r_d = gemv_case(TQ6, cfg2.wd, cfg2.h, H2, F2, copies=cfg2.copies)

        def step(i, nt):
            r_gu(i, nt)
            r_d(i, nt)
        record("cfg2_ffn_step", step, cfg2.step_bytes, None, budget, extra={"tier": orc.simd_tier(TQ4)})
        del gu
    # config 4: dense 512 tokens and the ragged batch (tokens/s)
    w4 = synth.make_weight(TQ8, 3584, 1024, seed=0, tag=TQ8)
    x4 = synth.make_act(1024, 512, seed=0, tag=400)
    record("cfg4_dense512_q8_0_3584x1024", gemv_case(TQ8, w4, x4, 3584, 1024), None, 512, budget,
           unit="tokens/s")
    lens = [int(v) for v in synth.ragged_lengths(8, 16, 256, seed=0)]
    xr = np.concatenate([synth.make_act(1024, n, seed=0, tag=300 + i) for i, n in enumerate(lens)])
    record("cfg4_ragged_q8_0_3584x1024", gemv_case(TQ8, w4, xr, 3584, 1024), None, sum(lens), budget,
           unit="tokens/s", extra={"tokens": sum(lens)})
    del w4, x4, xr
    # config 5: one and 64 tokens on both matrices
    for name, tt, rows, cols in (("cfg5_q4_k_17408x5120", TQ4, 17408, 5120), ("cfg5_q6_k_5120x17408", TQ6, 5120, 17408)):
        w5 = synth.make_weight(tt, rows, cols, seed=0, tag=tt)
        for T in (1, 64):
            x5 = synth.make_act(cols, T, seed=0, tag=500 + T)
            record(f"{name}_t{T}", gemv_case(tt, w5, x5, rows, cols), gemv_bytes(rows, cols, w5.nbytes, T), T,
                   budget / 2, unit="GB/s" if T == 1 else "tokens/s", extra={"tier": orc.simd_tier(tt)})
        del w5
    return res


# ---- the engine binding's buffers ---------------------------------------------------------

class HostMapped:
    """Pinned host memory mapped into the GPU (hipHostMalloc, mapped + coherent), as
    integration/backend_hip.zig allocates its Buf regions; dev is the device-side
    address from hipHostGetDevicePointer."""

    def __init__(self, nbytes: int):
        # the runtime torch and libqwen35_hip.so already share (same soname)
        self.hip = ctypes.CDLL("libamdhip64.so.7")
        self.hip.hipHostMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t, ctypes.c_uint]
        self.hip.hipHostGetDevicePointer.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p, ctypes.c_uint]
        self.hip.hipHostFree.argtypes = [ctypes.c_void_p]
        self.host = ctypes.c_void_p(0)
        rc = self.hip.hipHostMalloc(ctypes.byref(self.host), nbytes, 0x2 | 0x40000000)
        if rc != 0 or not self.host.value:
            raise RuntimeError(f"hipHostMalloc({nbytes}) failed: {rc}")
        self.dev = ctypes.c_void_p(0)
        rc = self.hip.hipHostGetDevicePointer(ctypes.byref(self.dev), self.host, 0)
        if rc != 0 or not self.dev.value:
            self.hip.hipHostFree(self.host)
            raise RuntimeError(f"hipHostGetDevicePointer failed: {rc}")
        self.nbytes = nbytes

    def numpy_f32(self, n: int):
        import numpy as np
        return np.ctypeslib.as_array((ctypes.c_float * n).from_address(self.host.value))

    def free(self):
        if self.host.value:
            self.hip.hipHostFree(self.host)
            self.host = ctypes.c_void_p(0)


def bench_binding(c: Ctx, c3: Cfg3, with_prefill: bool, iters: int = 200):
    """The matvec slot as integration/backend_hip.zig calls it: x and out in
    host-mapped Buf regions (the CPU slots around it read and write them), and
    a host wait after the launch.  Against the same slot on device buffers
    with the same wait, and with neither (the headline step).  Wall clock per
    slot call; host-side rates, never the headline value."""
    torch, lib = c.torch, c.lib

    def wall(fn, n):
        for _ in range(10):
            fn()
        t = time.perf_counter()
        for _ in range(n):
            fn()
        return (time.perf_counter() - t) / n

    xh, yh = HostMapped(4 * C3), HostMapped(4 * R3)
    try:
        xh.numpy_f32(C3)[:] = c3.x[0]
        lin = c3._lin

        def slot(out_p, x_p):
            def f():
                assert lib.qhip_backend_matvec(c3.be._h, out_p, lin, x_p) == 0
                assert lib.qhip_backend_sync(c3.be._h) == 0
            return f

        dev_s = wall(slot(c3._p[0], c3._p[1]), iters)
        host_s = wall(slot(yh.dev, xh.dev), iters)
        want = c3.y.cpu().numpy()
        got = yh.numpy_f32(R3)
        same = bool((got == want).all())
        res = {"cfg3_slot_us_device_bufs_with_wait": round(dev_s * 1e6, 2),
               "cfg3_slot_us_host_mapped_with_wait": round(host_s * 1e6, 2),
               "cfg3_host_mapped_gb_s": round(c3.alg / host_s / 1e9, 1),
               "host_mapped_output_equals_device_output": same,
               "note": "x (10 KB) is read and y (0.99 MB) written through the PCIe mapping; each slot waits "
                       "for its launch, as the binding's slots do"}
        log(f"binding: cfg3 slot {dev_s * 1e6:.1f} us on device buffers, {host_s * 1e6:.1f} us on host-mapped "
            f"x/out (both with the per-slot wait); outputs equal: {same}")
    finally:
        xh.free()
        yh.free()
    if not with_prefill:
        return res
    # a config-5 prefill slot: matvecBatchK of 512 tokens on the Q4_K gate
    # weight, 10.5 MB of x read and 35.7 MB of out written through the mapping
    T, rows, cols = 512, 17408, 5120
    be = c.ops.Backend(0)
    xh, yh = HostMapped(4 * T * cols), HostMapped(4 * T * rows)
    try:
        lin = be.load_linear(TQ4, rows, cols, c.synth.make_weight(TQ4, rows, cols, seed=0, tag=TQ4))
        be.prepare_linear(lin)
        x = c.synth.make_act(cols, T, seed=0, tag=500 + T)
        xh.numpy_f32(T * cols)[:] = x.reshape(-1)
        xd = torch.from_numpy(x).to(c.dev)
        yd = torch.empty((T, rows), device=c.dev)
        lp = ctypes.byref(lin)

        def bslot(out_p, x_p):
            def f():
                assert lib.qhip_backend_matvec_batch_k(be._h, out_p, lp, x_p, T) == 0
                assert lib.qhip_backend_sync(be._h) == 0
            return f

        bd = wall(bslot(ctypes.c_void_p(yd.data_ptr()), ctypes.c_void_p(xd.data_ptr())), 30)
        bh = wall(bslot(yh.dev, xh.dev), 30)
        same = bool((yh.numpy_f32(T * rows) == yd.cpu().numpy().reshape(-1)).all())
        res.update({"cfg5_q4k_t512_batch_us_device_bufs_with_wait": round(bd * 1e6, 2),
                    "cfg5_q4k_t512_batch_us_host_mapped_with_wait": round(bh * 1e6, 2),
                    "cfg5_host_mapped_output_equals_device_output": same})
        log(f"binding: cfg5 Q4_K matvecBatchK 512 tokens {bd * 1e6:.1f} us on device buffers, {bh * 1e6:.1f} us on "
            f"host-mapped x/out; outputs equal: {same}")
        be.free_linear(lin)
    finally:
        be.close()
        xh.free()
        yh.free()
    return res


# ---- profiling entry: one kernel only ---------------------------------------------------

def profile(c: Ctx, which: str, launches: int):
    torch, lib, ops, synth, dev, stream = c.torch, c.lib, c.ops, c.synth, c.dev, c.stream
    fn = None
    keep = []
    if which in ("cfg3_gemv", "cfg3_step", "cfg3_gemv_gguf"):
        c3 = Cfg3(c)
        keep.append(c3)
        fn = {"cfg3_gemv": c3.gemv, "cfg3_step": c3.step, "cfg3_gemv_gguf": c3.gemv_gguf}[which]
    elif which in ("cfg1_gemv", "cfg5_q4k_gemv", "cfg5_q6k_gemv", "cfg5_q6k_kimage"):
        tt, rows, cols = {"cfg1_gemv": (TQ8, 6144, 1024), "cfg5_q4k_gemv": (TQ4, 17408, 5120),
                          "cfg5_q6k_gemv": (TQ6, 5120, 17408), "cfg5_q6k_kimage": (TQ6, 5120, 17408)}[which]
        st, fn, k = gemv_stream(c, tt, rows, cols)
        keep += [st, k]
        if which == "cfg5_q6k_kimage":
            # the K-quant image of every rotated copy (what the Exec mirror
            # reads for one token), on the same pre-quantized activation
            imgs = [ops.gemv_image(tt, st.buf[j * st.stride:j * st.stride + st.n], rows, cols)
                    for j in range(st.copies)]
            aq, yo = k
            keep.append(imgs)

            def fn(i):
                assert lib.qhip_launch_mul_mat_vec_image(imgs[i % len(imgs)].data_ptr(), aq.data_ptr(),
                                                         yo.data_ptr(), rows, cols, tt, 0, stream) == 0
    elif which in ("down", "gate_up", "fused_gate_up", "split_down", "mirror_down", "step", "step_unfused"):
        c2 = Cfg2(c)
        keep.append(c2)
        fn = {"down": c2.gemv_down, "gate_up": c2.gemv_gate_up, "fused_gate_up": c2.fused_gate_up,
              "split_down": c2.split_down, "mirror_down": c2.down, "step": c2.step,
              "step_unfused": c2.step_unfused}[which]
    else:
        tt, rows, cols, T = {"mmq_cfg5_q4k": (TQ4, 17408, 5120, 512), "mmq_cfg5_q3k": (11, 17408, 5120, 512),
                             "mmq_cfg5_q2k": (10, 17408, 5120, 512), "mmq_cfg5_q6k_image": (TQ6, 5120, 17408, 512),
                             "mmq_cfg4": (TQ8, 3584, 1024, 512), "mmq_cfg5_q4k_frag": (TQ4, 17408, 5120, 512),
                             "mmq_cfg5_q4k_frag_t8": (TQ4, 17408, 5120, 8),
                             "mmq_cfg5_q6k_frag_t8": (TQ6, 5120, 17408, 8),
                             "mmq_cfg5_q6k_frag_t64": (TQ6, 5120, 17408, 64),
                             "mmq_cfg4_frag": (TQ8, 3584, 1024, 512),
                             "mmq_cfg4_ragged_frag": (TQ8, 3584, 1024, 0)}[which]
        w = torch.from_numpy(synth.make_weight(tt, rows, cols, seed=0, tag=tt)).to(dev)
        if which == "mmq_cfg4_ragged_frag":
            # the eight ragged sequences of bench_mmq, packed by the ragged quantizer
            lens = [int(v) for v in synth.ragged_lengths(8, 16, 256, seed=0)]
            seqs = [torch.from_numpy(synth.make_act(cols, n, seed=0, tag=300 + i)).to(dev) for i, n in enumerate(lens)]
            aq, off_d, T = ops.quantize_ragged(tt, seqs, cols)
            keep += seqs + [off_d]
        elif which == "mmq_cfg4_frag":
            aq = ops.quantize_act(tt, torch.from_numpy(synth.make_act(cols, T, seed=0, tag=400)).to(dev))
        else:
            aq = ops.quantize_act(tt, torch.from_numpy(synth.make_act(cols, T, seed=0, tag=500 + T)).to(dev))
        y = torch.empty((T, rows), device=dev)
        # the split-K workspace the Exec mirror passes
        wk = ops.mul_mat_work(rows, cols, T, tt, dev)
        wp, wn = (wk.data_ptr(), wk.numel()) if wk is not None else (None, 0)
        keep += [w, aq, y, wk]
        if which == "mmq_cfg5_q6k_image":
            img = ops.mmq_image(tt, w, rows, cols)
            keep.append(img)

            def fn(i):
                assert lib.qhip_launch_mul_mat_image(img.data_ptr(), aq.data_ptr(), y.data_ptr(), rows, cols, T, tt,
                                                     0, 0, wp, wn, stream) == 0
        elif which.startswith("mmq_cfg4_"):
            # the Q8_0 fragment image the Exec mirror reads for K <= 1024 (no workspace)
            img = ops.wd_image(tt, w, rows, cols)
            keep.append(img)

            def fn(i):
                assert lib.qhip_launch_mul_mat_wd_image(img.data_ptr(), aq.data_ptr(), y.data_ptr(), rows, cols, T,
                                                        tt, None, 0, stream) == 0
        elif "_frag" in which:
            # the fragment image the Exec mirror reads
            img = ops.wd_image(tt, w, rows, cols)
            keep.append(img)

            def fn(i):
                assert lib.qhip_launch_mul_mat_wd_image(img.data_ptr(), aq.data_ptr(), y.data_ptr(), rows, cols, T,
                                                        tt, wp, wn, stream) == 0
        else:
            def fn(i):
                assert lib.qhip_launch_mul_mat_work(w.data_ptr(), aq.data_ptr(), y.data_ptr(), rows, cols, T, tt,
                                                    PATH_MMQ, wp, wn, stream) == 0
    # the same warm-up and HIP-event timing as the measured run, so that a
    # trace of this process shows the launches bench.py reports: the last
    # `launches` launches of the kernel in the trace are the timed ones
    sec = time_loop(torch, fn, launches, 3)
    print(json.dumps({"profiled": which, "launches": launches, "event_avg_us": round(sec * 1e6, 3)}))


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="only the headline workload")
    ap.add_argument("--cpu-seconds", type=float, default=30.0, help="CPU baseline budget over all configs")
    ap.add_argument("--profile-kernel", choices=PROFILE_KERNELS, help="run only this kernel (for rocprofv3) and exit")
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
    c = Ctx(torch, np, lib, ops, synth, dev, torch.cuda.current_stream().cuda_stream)

    if args.copy_calib:
        n = 256 << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calib_bytes_read": n, "copy_calib_bytes_written": n, "launches": 5}))
        return 0
    if args.profile_kernel:
        profile(c, args.profile_kernel, args.steps)
        return 0

    # ---- headline: config 3 through the Exec mirror ------------------------------------
    c3 = Cfg3(c)
    sec = time_loop(torch, c3.step, args.steps, args.warmup)
    value = c3.alg / sec / 1e9
    log(f"cfg3 step (quantize + GEMV): {sec * 1e6:.2f} us, {value:.1f} GB/s ({100 * value / HBM_PEAK_GBS:.1f}% HBM)")
    n_k = max(200, args.steps)
    g_sec = time_loop(torch, c3.gemv, n_k, 20)
    q_sec = time_loop(torch, c3.quantize, n_k, 20)
    gg_sec = time_loop(torch, c3.gemv_gguf, n_k, 20)
    achieved = c3.alg / g_sec / 1e9
    kname = "gemv_image_iq4_nl_248320x2560"
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_for(kname), "kernel": kname,
                "alg_bytes_per_launch": c3.alg, "avg_launch_us": round(g_sec * 1e6, 3)}
    log(f"cfg3 image GEMV kernel alone: {g_sec * 1e6:.2f} us = {achieved:.1f} GB/s "
        f"({100 * achieved / HBM_PEAK_GBS:.1f}% of 8 TB/s); quantize launch {q_sec * 1e6:.2f} us; "
        f"GGUF-layout GEMV {gg_sec * 1e6:.2f} us")
    latency = {"cfg3_step_single_us": round(single_latency(torch, c3.step) * 1e6, 2),
               "cfg3_gemv_single_launch_us": round(single_latency(torch, c3.gemv) * 1e6, 2)}
    binding = bench_binding(c, c3, not args.no_extra)

    cfg2 = extra = mmq = None
    c2 = None
    if not args.no_extra:
        c2 = Cfg2(c)
        cfg2 = c2.run(args.steps, args.warmup)
        extra = bench_gemv_configs(c)
        mmq = bench_mmq(c)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(c, c3, c2, args.cpu_seconds, not args.no_extra)

    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(sec * 1e3, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (SplitMix64 seed 0, BASELINE.json config rules)",
        "config": {"workload": "cfg3: IQ4_NL output-head GEMV [248320,2560], batch 1, through the Exec mirror's "
                               "matvec from f32 x[2560] (Q8_0 quantization of x on the device, then the GEMV from "
                               "the weight's GEMV image, built at load time); 357 MB of weights resident in HBM, "
                               "larger than the Infinity Cache",
                   "hbm_frac": round(value / HBM_PEAK_GBS, 4), "step_alg_bytes": c3.alg,
                   "weight_sha256": c3.sha, "parallelism": "single GPU",
                   "gemv_kernel_us": round(g_sec * 1e6, 3), "quantize_launch_us": round(q_sec * 1e6, 3),
                   "gguf_layout_gemv_kernel_us": round(gg_sec * 1e6, 3)},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "latency": latency,
        "binding": binding,
        "cfg2_step": cfg2,
        "configs": extra,
        "mmq": mmq,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
