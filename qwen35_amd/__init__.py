"""qwen35_amd -- MI355X-native quantized GEMV / MMQ backend for qwen35.

The compute lives in libqwen35_hip.so (hand-written HIP for gfx950) behind
the C ABI in include/qwen35_hip.h.  This package only binds that ABI for
Python callers (tests, benchmarks); torch is used for device memory and
streams.
"""
from . import _lib
from ._lib import QhipError, QhipLinear, check, load

TT_Q8_0, TT_Q4_K, TT_Q6_K, TT_IQ4_NL = 8, 12, 14, 20
TT_Q2_K, TT_Q3_K, TT_Q5_K, TT_IQ4_XS = 10, 11, 13, 23
TT_Q4_0, TT_Q4_1 = 2, 3
TT_IQ3_XXS, TT_IQ3_S = 18, 21
PATH_AUTO, PATH_GEMV, PATH_MMQ, PATH_GENERIC = 0, 1, 2, 3
DECLINE = -1

__all__ = ["load", "check", "QhipError", "QhipLinear", "TT_Q8_0", "TT_Q4_K", "TT_Q6_K",
           "TT_IQ4_NL", "TT_Q2_K", "TT_Q3_K", "TT_Q5_K", "TT_IQ4_XS", "TT_Q4_0", "TT_Q4_1", "TT_IQ3_XXS", "TT_IQ3_S", "PATH_AUTO", "PATH_GEMV",
           "PATH_MMQ", "PATH_GENERIC", "DECLINE"]
