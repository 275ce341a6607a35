"""ctypes binding of libqwen35_hip.so (include/qwen35_hip.h).

Loading fails loudly when the library has not been built: there is no
fallback implementation of any entry point.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libqwen35_hip.so"

c_int, c_long, c_void_p, c_size_t = ctypes.c_int, ctypes.c_long, ctypes.c_void_p, ctypes.c_size_t
c_char_p = ctypes.c_char_p
c_int_p = ctypes.POINTER(ctypes.c_int)


class QhipLinear(ctypes.Structure):
    _fields_ = [("dev", c_void_p), ("ttype", c_int), ("rows", c_int), ("cols", c_int),
                ("row_bytes", c_long)]


class QhipProfEntry(ctypes.Structure):
    _fields_ = [("slot", c_int), ("ttype", c_int), ("rows", c_int), ("cols", c_int), ("tokens", c_int),
                ("calls", ctypes.c_longlong), ("device_us", ctypes.c_double), ("bytes", ctypes.c_double),
                ("ops", ctypes.c_double)]


# name: (restype, argtypes)
SIGNATURES = {
    "qhip_init": (c_int, [c_int]),
    "qhip_gpu_arch": (c_int, []),
    "qhip_gpu_cu_count": (c_int, []),
    "qhip_gpu_name": (c_char_p, []),
    "qhip_error_string": (c_char_p, [c_int]),
    "qhip_quant_act_block_elems": (c_int, [c_int]),
    "qhip_quant_geom": (c_int, [c_int, c_int_p, c_int_p]),
    "qhip_act_row_bytes": (c_long, [c_int, c_int]),
    "qhip_weight_row_bytes": (c_long, [c_int, c_int]),
    "qhip_launch_quantize_q8_0": (c_int, [c_void_p, c_void_p, c_int, c_void_p]),
    "qhip_launch_quantize_q8_K": (c_int, [c_void_p, c_void_p, c_int, c_void_p]),
    "qhip_launch_quantize_act": (c_int, [c_int, c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "qhip_launch_dequantize": (c_int, [c_int, c_void_p, c_void_p, c_int, c_void_p]),
    "qhip_launch_dequantize_row": (c_int, [c_int, c_void_p, c_void_p, c_int, c_void_p]),
    "qhip_launch_mul_mat_vec": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                                        c_void_p]),
    "qhip_launch_mul_mat_vec_q8_0": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int,
                                             c_void_p]),
    "qhip_launch_mul_mat": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                    c_void_p]),
    "qhip_launch_mul_mat_vec_tile": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                                             c_void_p]),
    "qhip_launch_mmq_tuned": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                      c_int, c_void_p]),
    "qhip_launch_quantize_mul_mat_vec": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int,
                                                 c_void_p]),
    "qhip_launch_quantize_mul_mat_vec_tuned": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                                       c_int, c_int, c_int, c_int, c_void_p]),
    "qhip_quantize_mul_mat_vec_work_bytes": (c_long, [c_int, c_int]),
    "qhip_launch_quantize_mul_mat_vec_split": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                                       c_int, c_int, c_int, c_int, c_void_p, c_long,
                                                       c_void_p]),
    "qhip_launch_quantize_mul_mat_vec_split_noalloc": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                                                               c_int, c_int, c_int, c_int, c_int, c_void_p]),
    "qhip_mmq_image_bytes": (c_long, [c_int, c_int, c_int]),
    "qhip_launch_mmq_prepare": (c_int, [c_int, c_void_p, c_int, c_int, c_void_p, c_void_p]),
    "qhip_launch_mul_mat_image": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                          c_int, c_void_p, c_long, c_void_p]),
    "qhip_wd_image_bytes": (c_long, [c_int, c_int, c_int]),
    "qhip_launch_wd_prepare": (c_int, [c_int, c_void_p, c_int, c_int, c_void_p, c_void_p]),
    "qhip_launch_mul_mat_wd_image": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p,
                                             c_long, c_void_p]),
    "qhip_gemv_image_bytes": (c_long, [c_int, c_int, c_int]),
    "qhip_gemv_image_act_bytes": (c_long, [c_int, c_int, c_int]),
    "qhip_launch_gemv_prepare": (c_int, [c_int, c_void_p, c_int, c_int, c_void_p, c_void_p]),
    "qhip_launch_quantize_act_image": (c_int, [c_int, c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "qhip_launch_mul_mat_vec_image": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p]),
    "qhip_mul_mat_work_bytes": (c_long, [c_int, c_int, c_int, c_int]),
    "qhip_launch_mul_mat_work": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                         c_void_p, c_long, c_void_p]),
    "qhip_launch_gemv_tuned": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                                       c_int, c_int, c_int, c_void_p]),
    "qhip_launch_quantize_ragged": (c_int, [c_int, c_void_p, c_void_p, c_int, c_int, c_int,
                                            c_void_p, c_void_p]),
    "qhip_ragged_offsets": (c_int, [c_int_p, c_int, c_int_p]),
    "qhip_launch_mul_mat_ragged": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p,
                                           c_int, c_int, c_int, c_void_p]),
    "qhip_launch_block_ints": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                                       c_void_p]),
    "qhip_backend_create": (c_void_p, [c_int, c_int_p]),
    "qhip_backend_destroy": (None, [c_void_p]),
    "qhip_backend_name": (c_char_p, [c_void_p]),
    "qhip_backend_load_linear": (c_int, [c_void_p, c_int, c_int, c_int, c_void_p,
                                         ctypes.POINTER(QhipLinear)]),
    "qhip_backend_wrap_linear": (c_int, [c_void_p, c_int, c_int, c_int, c_void_p,
                                         ctypes.POINTER(QhipLinear)]),
    "qhip_backend_free_linear": (None, [c_void_p, ctypes.POINTER(QhipLinear)]),
    "qhip_backend_prepare_linear": (c_int, [c_void_p, ctypes.POINTER(QhipLinear)]),
    "qhip_backend_set_mmq_images": (c_int, [c_void_p, c_int]),
    "qhip_backend_set_gemv_images": (c_int, [c_void_p, c_int]),
    "qhip_backend_set_mem_budget": (c_int, [c_void_p, c_size_t]),
    "qhip_backend_mem_placed": (c_size_t, [c_void_p]),
    "qhip_backend_alloc_scratch": (c_int, [c_void_p, c_int]),
    "qhip_backend_alloc_scratch_k": (c_int, [c_void_p, c_int, c_int]),
    "qhip_backend_free_scratch": (None, [c_void_p]),
    "qhip_backend_alloc_buf": (c_int, [c_void_p, c_size_t, ctypes.POINTER(c_void_p)]),
    "qhip_backend_matvec": (c_int, [c_void_p, c_void_p, ctypes.POINTER(QhipLinear), c_void_p]),
    "qhip_backend_matvec_pair": (c_int, [c_void_p, c_void_p, ctypes.POINTER(QhipLinear),
                                         ctypes.POINTER(QhipLinear), c_void_p]),
    "qhip_backend_matvec_batch_k": (c_int, [c_void_p, c_void_p, ctypes.POINTER(QhipLinear),
                                            c_void_p, c_int]),
    "qhip_backend_dequant_row": (c_int, [c_void_p, c_void_p, ctypes.POINTER(QhipLinear), c_int]),
    "qhip_backend_set_stream": (c_int, [c_void_p, c_void_p]),
    "qhip_backend_sync": (c_int, [c_void_p]),
    "qhip_backend_set_act_memo": (c_int, [c_void_p, c_int]),
    "qhip_backend_act_invalidate": (None, [c_void_p]),
    "qhip_backend_act_stats": (c_int, [c_void_p, ctypes.POINTER(ctypes.c_ulonglong),
                                       ctypes.POINTER(ctypes.c_ulonglong)]),
    "qhip_backend_step_begin": (None, [c_void_p, ctypes.c_uint]),
    "qhip_backend_step_end": (None, [c_void_p]),
    "qhip_backend_describe": (c_char_p, [c_void_p]),
    "qhip_backend_set_profiling": (c_int, [c_void_p, c_int]),
    "qhip_backend_prof_entries": (c_int, [c_void_p, ctypes.POINTER(QhipProfEntry), c_int]),
    "qhip_backend_prof_report": (c_long, [c_void_p, ctypes.c_char_p, c_long]),
    "qhip_backend_prof_untimed": (ctypes.c_longlong, [c_void_p]),
    "qhip_backend_prof_reset": (None, [c_void_p]),
}

_lib = None


def load(path: Path = LIB_PATH) -> ctypes.CDLL:
    """Load the HIP library (once).  Raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not path.exists():
        raise RuntimeError(
            f"{path} is missing: the HIP extension must be built "
            "(python -c 'import __graft_entry__ as g; g.build()'); there is no CPU fallback")
    lib = ctypes.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    _lib = lib
    return lib


class QhipError(RuntimeError):
    def __init__(self, what: str, code: int):
        lib = load()
        msg = lib.qhip_error_string(code)
        super().__init__(f"{what}: error {code} ({msg.decode() if msg else '?'})")
        self.code = code


def check(what: str, code: int) -> None:
    if code != 0:
        raise QhipError(what, code)
