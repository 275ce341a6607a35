"""C-ABI structure tests that need no GPU: the library loads, exports exactly
what include/qwen35_hip.h declares, and rejects bad arguments on the host
before any launch (the reference's host-side validation pattern,
src/kernels/cuda/mmvq.cu:781-785)."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "qwen35_hip.h"
INVALID = 1  # hipErrorInvalidValue


def declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(qhip_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    import qwen35_amd
    return qwen35_amd.load()


def test_header_declares_entry_points():
    names = declared()
    assert "qhip_launch_mul_mat_vec" in names and "qhip_backend_matvec_pair" in names
    assert len(names) >= 30


def test_library_exports_every_declared_symbol(lib):
    so = ROOT / "qwen35_amd" / "libqwen35_hip.so"
    out = subprocess.run(["nm", "-D", "--defined-only", str(so)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (qhip_\w+)", out))
    missing = [n for n in declared() if n not in exported]
    assert not missing, missing
    extra = sorted(exported - set(declared()))
    assert not extra, f"exported but undeclared: {extra}"


def test_python_binding_covers_header(lib):
    from qwen35_amd._lib import SIGNATURES
    assert sorted(SIGNATURES) == declared()


def test_geometry(lib):
    be, bb = ctypes.c_int(), ctypes.c_int()
    table = {8: (32, 34), 12: (256, 144), 14: (256, 210), 20: (32, 18), 13: (256, 176), 11: (256, 110),
             10: (256, 84), 23: (256, 136), 2: (32, 18), 3: (32, 20), 18: (256, 98), 21: (256, 110)}
    for tt, (e, b) in table.items():
        assert lib.qhip_quant_geom(tt, ctypes.byref(be), ctypes.byref(bb)) == 1
        assert (be.value, bb.value) == (e, b)
        assert lib.qhip_quant_act_block_elems(tt) == (32 if e == 32 else 256)
    assert lib.qhip_quant_geom(6, ctypes.byref(be), ctypes.byref(bb)) == 0  # Q5_0 unsupported
    assert lib.qhip_quant_geom(1, ctypes.byref(be), ctypes.byref(bb)) == 0  # F16: not a quant format
    assert lib.qhip_quant_act_block_elems(99) == 0
    assert lib.qhip_act_row_bytes(8, 1024) == 1088
    assert lib.qhip_act_row_bytes(12, 2560) == 2920
    assert lib.qhip_weight_row_bytes(14, 9728) == 7980
    assert lib.qhip_weight_row_bytes(20, 2560) == 1440
    assert lib.qhip_weight_row_bytes(12, 100) == -1  # not a multiple of 256
    assert lib.qhip_act_row_bytes(8, 48) == -1


def test_ragged_offsets(lib):
    lens = (ctypes.c_int * 4)(5, 0, 7, 3)
    off = (ctypes.c_int * 5)()
    assert lib.qhip_ragged_offsets(lens, 4, off) == 15
    assert list(off) == [0, 5, 5, 12, 15]
    bad = (ctypes.c_int * 2)(3, -1)
    assert lib.qhip_ragged_offsets(bad, 2, off) == -1


def test_invalid_arguments_rejected_before_launch(lib):
    p = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    # unknown type id
    assert lib.qhip_launch_mul_mat_vec(p, p, p, 16, 256, 1, 6, None) == INVALID
    # cols not a multiple of the block size
    assert lib.qhip_launch_mul_mat_vec(p, p, p, 16, 100, 1, 12, None) == INVALID
    # NULL buffers
    assert lib.qhip_launch_mul_mat_vec(None, p, p, 16, 256, 1, 8, None) == INVALID
    assert lib.qhip_launch_mul_mat_vec(p, None, p, 16, 256, 1, 8, None) == INVALID
    assert lib.qhip_launch_mul_mat_vec(p, p, None, 16, 256, 1, 8, None) == INVALID
    # negative counts
    assert lib.qhip_launch_mul_mat_vec(p, p, p, -1, 256, 1, 8, None) == INVALID
    assert lib.qhip_launch_mul_mat_vec(p, p, p, 16, 256, -2, 8, None) == INVALID
    # bad path selector
    assert lib.qhip_launch_mul_mat(p, p, p, 16, 256, 1, 8, 17, None) == INVALID
    # quantizers
    assert lib.qhip_launch_quantize_act(12, p, p, 100, 1, None) == INVALID
    assert lib.qhip_launch_quantize_act(8, None, p, 64, 1, None) == INVALID
    assert lib.qhip_launch_quantize_q8_0(None, p, 4, None) == INVALID
    assert lib.qhip_launch_quantize_q8_K(p, ctypes.c_void_p(0x1002), 1, None) == INVALID
    # ragged
    assert lib.qhip_launch_mul_mat_ragged(p, p, p, 16, 256, None, 2, 10, 8, None) == INVALID
    assert lib.qhip_launch_quantize_ragged(8, None, p, 2, 10, 256, p, None) == INVALID
    # parity export
    assert lib.qhip_launch_block_ints(p, p, p, 16, 96, 1, 8, None) == INVALID
    # one-launch quantize + GEMV: bad shapes, and the split-K workspace checks
    assert lib.qhip_launch_quantize_mul_mat_vec_tuned(p, p, None, p, 16, 256, 12, 65, 1, 256, None) == INVALID
    assert lib.qhip_launch_quantize_mul_mat_vec_tuned(p, p, None, p, 16, 256, 12, 8, 4, 1024, None) == INVALID
    need = lib.qhip_quantize_mul_mat_vec_work_bytes(16, 9728)
    assert lib.qhip_launch_quantize_mul_mat_vec_split(p, p, None, p, 16, 9728, 14, 0, 0, 0, None, need,
                                                      None) == INVALID
    assert lib.qhip_launch_quantize_mul_mat_vec_split(p, p, None, p, 16, 9728, 14, 0, 0, 0, p, need - 4,
                                                      None) == INVALID
    assert lib.qhip_launch_quantize_mul_mat_vec_split(p, p, None, p, 16, 9728, 14, 300, 0, 0, p, need,
                                                      None) == INVALID
    # GEMV image: formats without one, widths not a multiple of 64, alignment
    assert lib.qhip_gemv_image_bytes(13, 16, 2560) == -1
    assert lib.qhip_gemv_image_bytes(12, 16, 2560) == 16 * 1440   # Q4_K: the GGUF bytes reordered
    assert lib.qhip_gemv_image_bytes(14, 3, 2304) == 3 * 1890     # Q6_K
    assert lib.qhip_gemv_image_bytes(20, 16, 96) == -1
    assert lib.qhip_gemv_image_bytes(20, 16, 2560) == 16 * 1440
    assert lib.qhip_gemv_image_act_bytes(20, 2560, 2) == 2 * 72 * 40
    assert lib.qhip_gemv_image_act_bytes(8, 2560, 1) == 72 * 40  # Q8_0: the same split activation
    assert lib.qhip_gemv_image_bytes(8, 16, 2560) == 16 * 2720    # Q8_0: 68 bytes per 64 values
    assert lib.qhip_gemv_image_act_bytes(14, 2560, 2) == 2 * 292 * 10  # K-quants: the reference Q8_K rows
    assert lib.qhip_gemv_image_act_bytes(13, 2560, 1) == -1
    assert lib.qhip_launch_gemv_prepare(13, p, 16, 2560, ctypes.c_void_p(0x2000), None) == INVALID
    assert lib.qhip_launch_gemv_prepare(20, p, 16, 2560, ctypes.c_void_p(0x1008), None) == INVALID
    assert lib.qhip_launch_gemv_prepare(20, p, 16, 2560, p, None) == INVALID  # in place
    assert lib.qhip_launch_quantize_act_image(20, p, ctypes.c_void_p(0x1004), 2560, 1, None) == INVALID
    assert lib.qhip_launch_quantize_act_image(20, p, p, 96, 1, None) == INVALID
    assert lib.qhip_gemv_image_bytes(20, 16, 64) == -1      # no team width for one unit
    assert lib.qhip_gemv_image_bytes(20, 16, 9728) == -1    # long rows: the GGUF-layout kernels
    assert lib.qhip_launch_mul_mat_vec_image(p, p, p, 16, 2560, 20, 3, None) == INVALID
    assert lib.qhip_launch_mul_mat_vec_image(p, p, None, 16, 2560, 20, 0, None) == INVALID
    assert lib.qhip_launch_mul_mat_vec_image(p, p, p, 16, 2560, 13, 0, None) == INVALID
    assert lib.qhip_launch_mul_mat_vec_image(p, p, p, 16, 9728, 20, 0, None) == INVALID
    # fragment images: Q6_K, Q4_K, Q8_0; whole 256-value super-blocks; Q6_K 1..32 tokens; alignment
    assert lib.qhip_wd_image_bytes(14, 33, 512) == 2 * 2 * 6720
    assert lib.qhip_wd_image_bytes(14, 0, 512) == 0
    assert lib.qhip_wd_image_bytes(12, 33, 512) == 2 * 2 * 4608
    assert lib.qhip_wd_image_bytes(8, 33, 512) == 2 * 16 * 1088
    assert lib.qhip_wd_image_bytes(8, 32, 544) == -1
    assert lib.qhip_wd_image_bytes(2, 32, 512) == -1
    assert lib.qhip_wd_image_bytes(14, 32, 300) == -1
    assert lib.qhip_launch_wd_prepare(2, p, 32, 512, p, None) == INVALID
    assert lib.qhip_launch_wd_prepare(8, p, 32, 544, p, None) == INVALID
    assert lib.qhip_launch_wd_prepare(14, p, 32, 512, ctypes.c_void_p(0x1008), None) == INVALID
    assert lib.qhip_launch_mul_mat_wd_image(p, p, p, 32, 512, 65, 14, None, 0, None) == INVALID
    assert lib.qhip_launch_mul_mat_wd_image(p, p, p, 32, 512, 8, 2, None, 0, None) == INVALID
    assert lib.qhip_launch_mul_mat_wd_image(p, p, p, 32, 544, 8, 8, None, 0, None) == INVALID
    assert lib.qhip_launch_mul_mat_wd_image(ctypes.c_void_p(0x1008), p, p, 32, 512, 8, 14, None, 0,
                                            None) == INVALID
    assert lib.qhip_launch_mul_mat_wd_image(p, p, p, 32, 512, 8, 14, ctypes.c_void_p(0x1004), 4096,
                                            None) == INVALID
    assert lib.qhip_launch_mul_mat_wd_image(p, p, None, 32, 512, 8, 14, None, 0, None) == INVALID
    assert lib.qhip_launch_mul_mat_wd_image(p, p, p, 0, 512, 8, 14, None, 0, None) == 0
    # backend with bad handle
    assert lib.qhip_backend_set_gemv_images(None, 1) == INVALID
    assert lib.qhip_backend_matvec(None, p, None, p) == INVALID
    assert lib.qhip_backend_alloc_scratch(None, 1024) == INVALID


def test_split_workspace_size(lib):
    # 32 KiB of row-tile counters, then one f32 partial per row and 256-value slice
    for rows, cols in [(2560, 9728), (1, 256), (5120, 17408), (7, 300)]:
        assert lib.qhip_quantize_mul_mat_vec_work_bytes(rows, cols) == 32768 + 4 * rows * ((cols + 255) // 256)
    assert lib.qhip_quantize_mul_mat_vec_work_bytes(-1, 256) == 0


def test_mmq_split_workspace_size(lib):
    # cfg5 at 16 tokens splits K (a few hundred row tiles).  From one round of
    # resident weights-direct tiles (512 workgroups), the whole rounds stay
    # whole and only the last, partial round's tiles are cut over K (20
    # super-blocks): 256 tokens, 544 tiles, the last 32 in 10 slices; 512
    # tokens, 1088 tiles, the last 64 in 7; 1024 tokens, 2176 tiles, the last
    # 128 in 4.  A GEMV-only or unknown type has no workspace
    n = lib.qhip_mul_mat_work_bytes(17408, 5120, 16, 12)
    assert n > 32768 and n % 4 == 0
    assert lib.qhip_mul_mat_work_bytes(5120, 17408, 16, 14) > 32768
    assert lib.qhip_mul_mat_work_bytes(17408, 5120, 256, 12) == 32768 + 4 * 10 * 32 * 64 * 128
    assert lib.qhip_mul_mat_work_bytes(17408, 5120, 512, 12) == 32768 + 4 * 7 * 64 * 64 * 128
    assert lib.qhip_mul_mat_work_bytes(17408, 5120, 1024, 12) == 32768 + 4 * 4 * 128 * 64 * 128
    assert lib.qhip_mul_mat_work_bytes(17408, 5120, 16, 99) == 0
    assert lib.qhip_mul_mat_work_bytes(0, 5120, 16, 12) == 0
    p = ctypes.c_void_p(0x1000)
    # a misaligned workspace or a negative size is rejected before any launch
    assert lib.qhip_launch_mul_mat_work(p, p, p, 16, 256, 8, 12, 0, ctypes.c_void_p(0x1004), n, None) == INVALID
    assert lib.qhip_launch_mul_mat_work(p, p, p, 16, 256, 8, 12, 0, p, -1, None) == INVALID
    assert lib.qhip_launch_mul_mat_image(p, p, p, 16, 256, 8, 12, 0, 0, ctypes.c_void_p(0x1004), n,
                                         None) == INVALID


def test_zero_sized_requests_are_no_ops(lib):
    p = ctypes.c_void_p(0x1000)
    assert lib.qhip_launch_mul_mat_vec(p, p, p, 0, 256, 1, 8, None) == 0
    assert lib.qhip_launch_mul_mat_vec(p, p, p, 16, 256, 0, 8, None) == 0
    assert lib.qhip_launch_quantize_act(8, p, p, 64, 0, None) == 0


def test_error_strings(lib):
    assert b"declined" in lib.qhip_error_string(-1)


def test_missing_library_fails_loudly(tmp_path):
    from qwen35_amd import _lib
    saved = _lib._lib
    try:
        _lib._lib = None
        with pytest.raises(RuntimeError, match="no CPU fallback"):
            _lib.load(tmp_path / "absent.so")
    finally:
        _lib._lib = saved
