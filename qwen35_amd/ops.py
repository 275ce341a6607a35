"""Thin torch-facing wrappers over the C ABI (device tensors in, device tensors out).

Every call goes straight to a HIP kernel of libqwen35_hip.so on the current
torch stream; nothing is computed on the host.
"""
from __future__ import annotations

import ctypes

import torch

from ._lib import QhipLinear, QhipProfEntry, check, load

_GEOM = {8: (32, 34), 20: (32, 18), 12: (256, 144), 14: (256, 210), 13: (256, 176), 11: (256, 110),
         10: (256, 84), 23: (256, 136), 2: (32, 18), 3: (32, 20), 18: (256, 98), 21: (256, 110)}
# integers per 32-value block in the block-integer export: (sumi, sumy) for Q4_1
_NINTS_32 = {3: 2}
# integers per super-block in the block-integer export: (isum, summs) for
# Q4_K / Q5_K / Q2_K, one per 32-value block for IQ4_XS and the IQ3 formats, else one
_NINTS_SB = {12: 2, 13: 2, 10: 2, 23: 8, 18: 8, 21: 8}


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _p(t: torch.Tensor) -> ctypes.c_void_p:
    assert t.is_cuda and t.is_contiguous()
    return ctypes.c_void_p(t.data_ptr())


def act_row_bytes(ttype: int, cols: int) -> int:
    n = load().qhip_act_row_bytes(ttype, cols)
    if n < 0:
        raise ValueError(f"bad (ttype={ttype}, cols={cols})")
    return n


def weight_row_bytes(ttype: int, cols: int) -> int:
    n = load().qhip_weight_row_bytes(ttype, cols)
    if n < 0:
        raise ValueError(f"bad (ttype={ttype}, cols={cols})")
    return n


def quantize_act(ttype: int, x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """x [k, cols] f32 -> [k, act_row_bytes] uint8, the weight type's activation family."""
    x2 = x.reshape(-1, x.shape[-1])
    k, cols = x2.shape
    if out is None:
        out = torch.empty((k, act_row_bytes(ttype, cols)), dtype=torch.uint8, device=x.device)
    check("quantize_act", load().qhip_launch_quantize_act(ttype, _p(x2), _p(out), cols, k, _stream()))
    return out


def quantize_q8_0(x: torch.Tensor) -> torch.Tensor:
    n = x.numel()
    out = torch.empty(n // 32 * 34, dtype=torch.uint8, device=x.device)
    check("quantize_q8_0", load().qhip_launch_quantize_q8_0(_p(x), _p(out), n // 32, _stream()))
    return out


def quantize_q8_K(x: torch.Tensor) -> torch.Tensor:
    n = x.numel()
    out = torch.empty(n // 256 * 292, dtype=torch.uint8, device=x.device)
    check("quantize_q8_K", load().qhip_launch_quantize_q8_K(_p(x), _p(out), n // 256, _stream()))
    return out


def dequantize(ttype: int, w: torch.Tensor, nblocks: int) -> torch.Tensor:
    """f32 values of `nblocks` native blocks (bit-exact with the reference dequant)."""
    be = _GEOM[ttype][0]
    out = torch.empty(nblocks * be, dtype=torch.float32, device=w.device)
    check("dequantize", load().qhip_launch_dequantize(ttype, _p(w), _p(out), nblocks, _stream()))
    return out


def dequantize_row(ttype: int, wrow: torch.Tensor, cols: int) -> torch.Tensor:
    out = torch.empty(cols, dtype=torch.float32, device=wrow.device)
    check("dequantize_row", load().qhip_launch_dequantize_row(ttype, _p(wrow), _p(out), cols, _stream()))
    return out


def mul_mat(ttype: int, w: torch.Tensor, xq: torch.Tensor, rows: int, cols: int, tokens: int,
            path: int = 0, out: torch.Tensor | None = None) -> torch.Tensor:
    """out [tokens, rows] = W . xq_t (xq already quantized)."""
    if out is None:
        out = torch.empty((tokens, rows), dtype=torch.float32, device=w.device)
    check("mul_mat", load().qhip_launch_mul_mat(_p(w), _p(xq), _p(out), rows, cols, tokens, ttype,
                                                path, _stream()))
    return out


def mul_mat_work(rows: int, cols: int, tokens: int, ttype: int, device) -> torch.Tensor | None:
    """Zeroed split-K workspace for mul_mat_split / mul_mat_image (None when no split would be made)."""
    n = load().qhip_mul_mat_work_bytes(rows, cols, tokens, ttype)
    return torch.zeros(n, dtype=torch.uint8, device=device) if n > 0 else None


def mul_mat_split(ttype: int, w: torch.Tensor, xq: torch.Tensor, rows: int, cols: int, tokens: int,
                  work: torch.Tensor | None, path: int = 0, out: torch.Tensor | None = None) -> torch.Tensor:
    """mul_mat with a workspace: the MMQ of small grids splits K (deterministic slice order)."""
    if out is None:
        out = torch.empty((tokens, rows), dtype=torch.float32, device=w.device)
    check("mul_mat_work", load().qhip_launch_mul_mat_work(
        _p(w), _p(xq), _p(out), rows, cols, tokens, ttype, path, _p(work) if work is not None else None,
        work.numel() if work is not None else 0, _stream()))
    return out


def quantize_mul_mat_vec(ttype: int, w: torch.Tensor, x: torch.Tensor, rows: int, cols: int,
                         xq_out: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """One launch: quantize f32 x (one token) inside the GEMV and multiply."""
    if out is None:
        out = torch.empty(rows, dtype=torch.float32, device=w.device)
    check("quantize_mul_mat_vec", load().qhip_launch_quantize_mul_mat_vec(
        _p(w), _p(x), _p(xq_out) if xq_out is not None else None, _p(out), rows, cols, ttype, _stream()))
    return out


def quantize_mul_mat_vec_tuned(ttype: int, w: torch.Tensor, x: torch.Tensor, rows: int, cols: int,
                               lanes_per_row: int = 0, rows_per_lane: int = 0, workgroup_threads: int = 0,
                               xq_out: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """The one-launch quantize + GEMV with an explicit shape (0 = pick)."""
    if out is None:
        out = torch.empty(rows, dtype=torch.float32, device=w.device)
    check("quantize_mul_mat_vec_tuned", load().qhip_launch_quantize_mul_mat_vec_tuned(
        _p(w), _p(x), _p(xq_out) if xq_out is not None else None, _p(out), rows, cols, ttype, lanes_per_row,
        rows_per_lane, workgroup_threads, _stream()))
    return out


def split_work(rows: int, cols: int, device) -> torch.Tensor:
    """Zeroed workspace for quantize_mul_mat_vec_split (its counters must start at zero)."""
    n = load().qhip_quantize_mul_mat_vec_work_bytes(rows, cols)
    return torch.zeros(max(n, 16), dtype=torch.uint8, device=device)


def quantize_mul_mat_vec_split(ttype: int, w: torch.Tensor, x: torch.Tensor, rows: int, cols: int,
                               work: torch.Tensor, slice_values: int = 0, lanes_per_row: int = 0,
                               rows_per_lane: int = 0, xq_out: torch.Tensor | None = None,
                               out: torch.Tensor | None = None) -> torch.Tensor:
    """One launch, split over K: each workgroup quantizes and multiplies one slice of x."""
    if out is None:
        out = torch.empty(rows, dtype=torch.float32, device=w.device)
    check("quantize_mul_mat_vec_split", load().qhip_launch_quantize_mul_mat_vec_split(
        _p(w), _p(x), _p(xq_out) if xq_out is not None else None, _p(out), rows, cols, ttype, slice_values,
        lanes_per_row, rows_per_lane, _p(work), work.numel(), _stream()))
    return out


def quantize_mul_mat_vec_split_noalloc(ttype: int, w: torch.Tensor, x: torch.Tensor, rows: int, cols: int,
                                       slice_values: int = 0, lanes_per_row: int = 0, rows_per_lane: int = 0,
                                       xq_out: torch.Tensor | None = None,
                                       out: torch.Tensor | None = None) -> torch.Tensor:
    """The split-K launch with the library's own per-device workspace (no allocation in the call)."""
    if out is None:
        out = torch.empty(rows, dtype=torch.float32, device=w.device)
    check("quantize_mul_mat_vec_split_noalloc", load().qhip_launch_quantize_mul_mat_vec_split_noalloc(
        _p(w), _p(x), _p(xq_out) if xq_out is not None else None, _p(out), rows, cols, ttype, slice_values,
        lanes_per_row, rows_per_lane, _stream()))
    return out


def gemv_tuned(ttype: int, w: torch.Tensor, xq: torch.Tensor, rows: int, cols: int, tokens: int,
               lanes_per_row: int, tokens_per_pass: int, rows_per_lane: int = 1,
               out: torch.Tensor | None = None) -> torch.Tensor:
    if out is None:
        out = torch.empty((tokens, rows), dtype=torch.float32, device=w.device)
    check("gemv_tuned", load().qhip_launch_gemv_tuned(_p(w), _p(xq), _p(out), rows, cols, tokens,
                                                      ttype, lanes_per_row, tokens_per_pass,
                                                      rows_per_lane, _stream()))
    return out


def mmq_tuned(ttype: int, w: torch.Tensor, xq: torch.Tensor, rows: int, cols: int, tokens: int,
              tile_tokens: int = 0, tile_rows: int = 0, out: torch.Tensor | None = None) -> torch.Tensor:
    """The int8-MFMA tile path with an explicit workgroup tile (64 or 128 each, 0 = pick)."""
    if out is None:
        out = torch.empty((tokens, rows), dtype=torch.float32, device=w.device)
    check("mmq_tuned", load().qhip_launch_mmq_tuned(_p(w), _p(xq), _p(out), rows, cols, tokens, ttype,
                                                    tile_tokens, tile_rows, _stream()))
    return out


def mmq_image(ttype: int, w: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    """The MMQ weight image of a Q4_K / Q6_K weight (sub-scales folded into two int8 planes)."""
    n = load().qhip_mmq_image_bytes(ttype, rows, cols)
    if n < 0:
        raise ValueError(f"no MMQ image for type {ttype} at cols={cols}")
    img = torch.empty(max(n, 16), dtype=torch.uint8, device=w.device)
    check("mmq_prepare", load().qhip_launch_mmq_prepare(ttype, _p(w), rows, cols, _p(img), _stream()))
    return img


def mul_mat_image(ttype: int, img: torch.Tensor, xq: torch.Tensor, rows: int, cols: int, tokens: int,
                  tile_tokens: int = 0, tile_rows: int = 0, work: torch.Tensor | None = None) -> torch.Tensor:
    out = torch.empty((tokens, rows), dtype=torch.float32, device=img.device)
    check("mul_mat_image", load().qhip_launch_mul_mat_image(
        _p(img), _p(xq), _p(out), rows, cols, tokens, ttype, tile_tokens, tile_rows,
        _p(work) if work is not None else None, work.numel() if work is not None else 0, _stream()))
    return out


def wd_image(ttype: int, w: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    """The fragment image of a Q4_K / Q6_K / Q8_0 weight (the GGUF bytes permuted for the MMQ)."""
    n = load().qhip_wd_image_bytes(ttype, rows, cols)
    if n < 0:
        raise ValueError(f"no fragment image for type {ttype} at cols={cols}")
    img = torch.empty(max(n, 16), dtype=torch.uint8, device=w.device)
    check("wd_prepare", load().qhip_launch_wd_prepare(ttype, _p(w), rows, cols, _p(img), _stream()))
    return img


def mul_mat_wd_image(ttype: int, img: torch.Tensor, xq: torch.Tensor, rows: int, cols: int, tokens: int,
                     work: torch.Tensor | None = None) -> torch.Tensor:
    """out [tokens, rows] from the fragment image (Q6_K: 1..32 tokens; Q4_K, Q8_0: any)."""
    out = torch.empty((tokens, rows), dtype=torch.float32, device=img.device)
    check("mul_mat_wd_image", load().qhip_launch_mul_mat_wd_image(
        _p(img), _p(xq), _p(out), rows, cols, tokens, ttype,
        _p(work) if work is not None else None, work.numel() if work is not None else 0, _stream()))
    return out


def gemv_image(ttype: int, w: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    """The GEMV weight image of an IQ4_NL / Q4_0 weight (same bytes per row, quant bytes 16-byte aligned)."""
    n = load().qhip_gemv_image_bytes(ttype, rows, cols)
    if n < 0:
        raise ValueError(f"no GEMV image for type {ttype} at cols={cols}")
    img = torch.empty(max(n, 16), dtype=torch.uint8, device=w.device)
    check("gemv_prepare", load().qhip_launch_gemv_prepare(ttype, _p(w), rows, cols, _p(img), _stream()))
    return img


def quantize_act_image(ttype: int, x: torch.Tensor) -> torch.Tensor:
    """f32 [tokens, cols] -> the split Q8_0 activation the GEMV image reads."""
    x = x.contiguous()
    cols = x.shape[-1]
    tokens = x.numel() // cols
    n = load().qhip_gemv_image_act_bytes(ttype, cols, tokens)
    if n < 0:
        raise ValueError(f"no split activation for type {ttype} at cols={cols}")
    out = torch.empty(max(n, 16), dtype=torch.uint8, device=x.device)
    check("quantize_act_image", load().qhip_launch_quantize_act_image(ttype, _p(x), _p(out), cols, tokens,
                                                                      _stream()))
    return out


def mul_mat_vec_image(ttype: int, img: torch.Tensor, xa: torch.Tensor, rows: int, cols: int,
                      rows_per_lane: int = 0) -> torch.Tensor:
    out = torch.empty(rows, dtype=torch.float32, device=img.device)
    check("mul_mat_vec_image", load().qhip_launch_mul_mat_vec_image(
        _p(img), _p(xa), _p(out), rows, cols, ttype, rows_per_lane, _stream()))
    return out


def block_ints(ttype: int, w: torch.Tensor, xq: torch.Tensor, rows: int, cols: int,
               tokens: int) -> torch.Tensor:
    be = _GEOM[ttype][0]
    nints = _NINTS_32.get(ttype, 1) * (cols // 32) if be == 32 else _NINTS_SB.get(ttype, 1) * (cols // 256)
    out = torch.empty((tokens, rows, nints), dtype=torch.int32, device=w.device)
    check("block_ints", load().qhip_launch_block_ints(_p(w), _p(xq), _p(out), rows, cols, tokens,
                                                      ttype, _stream()))
    return out


def ragged_offsets(lengths) -> tuple[list[int], int]:
    n = len(lengths)
    arr = (ctypes.c_int * n)(*lengths)
    off = (ctypes.c_int * (n + 1))()
    total = load().qhip_ragged_offsets(arr, n, off)
    if total < 0:
        raise ValueError("bad lengths")
    return list(off), total


def quantize_ragged(ttype: int, seqs: list[torch.Tensor], cols: int):
    """Pack + quantize several [L_i, cols] f32 sequences in one launch.
    Returns (xq_packed [total, act_row_bytes], offsets_dev [nseq+1] int32, total)."""
    lengths = [int(s.shape[0]) for s in seqs]
    off, total = ragged_offsets(lengths)
    dev = seqs[0].device
    ptrs = torch.tensor([s.data_ptr() for s in seqs], dtype=torch.int64, device=dev)
    off_d = torch.tensor(off, dtype=torch.int32, device=dev)
    xq = torch.empty((max(total, 1), act_row_bytes(ttype, cols)), dtype=torch.uint8, device=dev)
    check("quantize_ragged", load().qhip_launch_quantize_ragged(
        ttype, _p(ptrs), _p(off_d), len(seqs), total, cols, _p(xq), _stream()))
    return xq, off_d, total


def mul_mat_ragged(ttype: int, w: torch.Tensor, xq: torch.Tensor, off_d: torch.Tensor, nseq: int,
                   total: int, rows: int, cols: int) -> torch.Tensor:
    out = torch.empty((max(total, 1), rows), dtype=torch.float32, device=w.device)
    check("mul_mat_ragged", load().qhip_launch_mul_mat_ragged(
        _p(w), _p(xq), _p(out), rows, cols, _p(off_d), nseq, total, ttype, _stream()))
    return out[:total]


class Backend:
    """Python handle on the C++ backend (the Exec-slot mirror)."""

    def __init__(self, device: int = 0):
        lib = load()
        err = ctypes.c_int(0)
        self._h = lib.qhip_backend_create(device, ctypes.byref(err))
        if not self._h:
            check("backend_create", err.value or -1)
        self.lib = lib
        check("set_stream", lib.qhip_backend_set_stream(self._h, _stream()))

    def close(self):
        if self._h:
            self.lib.qhip_backend_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def name(self) -> str:
        return self.lib.qhip_backend_name(self._h).decode()

    def load_linear(self, ttype: int, rows: int, cols: int, host_bytes) -> QhipLinear:
        import numpy as np
        buf = np.ascontiguousarray(host_bytes, dtype=np.uint8)
        lin = QhipLinear()
        check("load_linear", self.lib.qhip_backend_load_linear(
            self._h, ttype, rows, cols, ctypes.c_void_p(buf.ctypes.data), ctypes.byref(lin)))
        return lin

    def wrap_linear(self, ttype: int, rows: int, cols: int, dev: torch.Tensor) -> QhipLinear:
        lin = QhipLinear()
        check("wrap_linear", self.lib.qhip_backend_wrap_linear(self._h, ttype, rows, cols, _p(dev),
                                                               ctypes.byref(lin)))
        return lin

    def free_linear(self, w: QhipLinear) -> None:
        self.lib.qhip_backend_free_linear(self._h, ctypes.byref(w))

    def prepare_linear(self, w: QhipLinear) -> int:
        """Build the weight's GEMV / MMQ image now: 0 built / nothing to build, -1 not built."""
        rc = self.lib.qhip_backend_prepare_linear(self._h, ctypes.byref(w))
        if rc not in (0, -1):
            check("prepare_linear", rc)
        return rc

    def set_mmq_images(self, on: bool) -> None:
        check("set_mmq_images", self.lib.qhip_backend_set_mmq_images(self._h, int(bool(on))))

    def set_gemv_images(self, on: bool) -> None:
        check("set_gemv_images", self.lib.qhip_backend_set_gemv_images(self._h, int(bool(on))))

    def set_mem_budget(self, nbytes: int) -> None:
        check("set_mem_budget", self.lib.qhip_backend_set_mem_budget(self._h, nbytes))

    def mem_placed(self) -> int:
        return int(self.lib.qhip_backend_mem_placed(self._h))

    def matvec(self, out: torch.Tensor, w: QhipLinear, x: torch.Tensor) -> None:
        check("matvec", self.lib.qhip_backend_matvec(self._h, _p(out), ctypes.byref(w), _p(x)))

    def matvec_pair(self, out: torch.Tensor, a: QhipLinear, b: QhipLinear, x: torch.Tensor) -> None:
        check("matvec_pair", self.lib.qhip_backend_matvec_pair(self._h, _p(out), ctypes.byref(a),
                                                               ctypes.byref(b), _p(x)))

    def matvec_batch_k(self, out: torch.Tensor, w: QhipLinear, xk: torch.Tensor, k: int) -> None:
        check("matvec_batch_k", self.lib.qhip_backend_matvec_batch_k(self._h, _p(out),
                                                                     ctypes.byref(w), _p(xk), k))

    def dequant_row(self, out: torch.Tensor, w: QhipLinear, row: int) -> None:
        check("dequant_row", self.lib.qhip_backend_dequant_row(self._h, _p(out), ctypes.byref(w), row))

    def sync(self) -> None:
        check("sync", self.lib.qhip_backend_sync(self._h))

    def set_stream(self, stream) -> None:
        """Launch on `stream` (a torch stream or a raw handle) from now on."""
        h = getattr(stream, "cuda_stream", stream)
        check("set_stream", self.lib.qhip_backend_set_stream(self._h, ctypes.c_void_p(h)))

    def set_act_memo(self, on: bool) -> None:
        check("set_act_memo", self.lib.qhip_backend_set_act_memo(self._h, int(bool(on))))

    def act_invalidate(self) -> None:
        self.lib.qhip_backend_act_invalidate(self._h)

    def act_stats(self) -> tuple[int, int]:
        hits, misses = ctypes.c_ulonglong(0), ctypes.c_ulonglong(0)
        check("act_stats", self.lib.qhip_backend_act_stats(self._h, ctypes.byref(hits),
                                                           ctypes.byref(misses)))
        return hits.value, misses.value

    def step_begin(self, pos: int) -> None:
        self.lib.qhip_backend_step_begin(self._h, pos)

    def step_end(self) -> None:
        self.lib.qhip_backend_step_end(self._h)

    def describe(self) -> str:
        return self.lib.qhip_backend_describe(self._h).decode()

    def set_profiling(self, on: bool) -> None:
        check("set_profiling", self.lib.qhip_backend_set_profiling(self._h, int(bool(on))))

    def prof_entries(self) -> list[dict]:
        """The device-time table, largest total first (waits for outstanding timings)."""
        n = self.lib.qhip_backend_prof_entries(self._h, None, 0)
        check("prof_entries", 0 if n >= 0 else n)
        arr = (QhipProfEntry * max(n, 1))()
        m = self.lib.qhip_backend_prof_entries(self._h, arr, n)
        assert m == n
        return [{f: getattr(arr[i], f) for f, _ in QhipProfEntry._fields_} for i in range(n)]

    def prof_report(self) -> str:
        n = self.lib.qhip_backend_prof_report(self._h, None, 0)
        assert n >= 0
        buf = ctypes.create_string_buffer(n + 1)
        assert self.lib.qhip_backend_prof_report(self._h, buf, n + 1) == n
        return buf.value.decode()

    def prof_untimed(self) -> int:
        return int(self.lib.qhip_backend_prof_untimed(self._h))

    def prof_reset(self) -> None:
        self.lib.qhip_backend_prof_reset(self._h)
