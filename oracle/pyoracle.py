"""ctypes view of the CPU checker (oracle/liboracle.so) and of the reference's
own compiled kernels (oracle/_ref/libqref.so, when built).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py.  The shipped package never imports this module.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# QWEN35_ORACLE_SO names another build of the same restatement (the sanitized
# one, oracle/_san/liboracle.so)
ORACLE_SO = Path(os.environ.get("QWEN35_ORACLE_SO") or HERE / "liboracle.so")
REF_SO = HERE / "_ref" / "libqref.so"

TT_Q8_0, TT_Q4_K, TT_Q6_K, TT_IQ4_NL = 8, 12, 14, 20
TT_Q2_K, TT_Q3_K, TT_Q5_K, TT_IQ4_XS = 10, 11, 13, 23
TT_Q4_0, TT_Q4_1 = 2, 3
TT_IQ3_XXS, TT_IQ3_S = 18, 21
GEOM = {TT_Q8_0: (32, 34), TT_IQ4_NL: (32, 18), TT_Q4_K: (256, 144), TT_Q6_K: (256, 210),
        TT_Q2_K: (256, 84), TT_Q3_K: (256, 110), TT_Q5_K: (256, 176), TT_IQ4_XS: (256, 136),
        TT_Q4_0: (32, 18), TT_Q4_1: (32, 20), TT_IQ3_XXS: (256, 98), TT_IQ3_S: (256, 110)}
NAMES = {TT_Q8_0: "Q8_0", TT_Q4_K: "Q4_K", TT_Q6_K: "Q6_K", TT_IQ4_NL: "IQ4_NL",
         TT_Q2_K: "Q2_K", TT_Q3_K: "Q3_K", TT_Q5_K: "Q5_K", TT_IQ4_XS: "IQ4_XS",
         TT_Q4_0: "Q4_0", TT_Q4_1: "Q4_1", TT_IQ3_XXS: "IQ3_XXS", TT_IQ3_S: "IQ3_S"}
# the formats of the benchmark configurations, the further K-quant family, the
# legacy 32-value formats (Q8_0 activations) and the 3-bit grid formats of real
# GGUF files
BASE_TYPES = [TT_Q8_0, TT_Q4_K, TT_Q6_K, TT_IQ4_NL]
EXTRA_TYPES = [TT_Q5_K, TT_Q3_K, TT_Q2_K, TT_IQ4_XS, TT_Q4_0, TT_Q4_1, TT_IQ3_XXS, TT_IQ3_S]
ALL_TYPES = BASE_TYPES + EXTRA_TYPES
# integers per weight block in block_ints: (isum, summs) for the K-quants with
# mins, (sumi, sumy) for Q4_1, one per 32-value block (before its scale) for
# IQ4_XS and the IQ3 formats, else one
NINTS = {TT_Q4_K: 2, TT_Q5_K: 2, TT_Q2_K: 2, TT_IQ4_XS: 8, TT_Q4_1: 2, TT_IQ3_XXS: 8, TT_IQ3_S: 8}

_c_u8p = ctypes.POINTER(ctypes.c_uint8)
_c_f32p = ctypes.POINTER(ctypes.c_float)
_c_i32p = ctypes.POINTER(ctypes.c_int32)
DOT_FN = ctypes.CFUNCTYPE(ctypes.c_float, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p)
QUANT_FN = ctypes.CFUNCTYPE(None, ctypes.c_int, _c_f32p, _c_u8p)


def _ptr(a: np.ndarray, t=ctypes.c_void_p):
    assert a.flags["C_CONTIGUOUS"]
    return ctypes.cast(a.ctypes.data, t)


def act_block_elems(ttype: int) -> int:
    return 32 if GEOM[ttype][0] == 32 else 256


def act_bytes(ttype: int, cols: int) -> int:
    return cols // 32 * 34 if act_block_elems(ttype) == 32 else cols // 256 * 292


def row_bytes(ttype: int, cols: int) -> int:
    be, bb = GEOM[ttype]
    return cols // be * bb


class Oracle:
    """The repository's C restatement of the reference arithmetic."""

    def __init__(self, path: Path = ORACLE_SO):
        if not path.exists():
            raise FileNotFoundError(f"{path} not built (run __graft_entry__.build())")
        L = self.lib = ctypes.CDLL(str(path))
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_dot.restype = ctypes.c_float
        L.orc_dot.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
        L.orc_row_block_ints.restype = ctypes.c_int
        L.orc_row_block_ints.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                         ctypes.c_void_p, _c_i32p]
        L.orc_quantize_act.restype = ctypes.c_int
        L.orc_quantize_act.argtypes = [ctypes.c_int, ctypes.c_int, _c_f32p, _c_u8p]
        L.orc_matvec_batch.restype = ctypes.c_int
        L.orc_matvec_batch.argtypes = [ctypes.c_int] * 4 + [ctypes.c_void_p, _c_f32p, _c_f32p,
                                                            ctypes.c_int]
        L.orc_matvec_q_fn.restype = ctypes.c_int
        L.orc_matvec_q_fn.argtypes = [ctypes.c_void_p] + [ctypes.c_int] * 4 + [
            ctypes.c_void_p, ctypes.c_void_p, _c_f32p, ctypes.c_int]
        L.orc_matvec_batch_fn.restype = ctypes.c_int
        L.orc_matvec_batch_fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int] * 4 + [
            ctypes.c_void_p, _c_f32p, _c_f32p, _c_u8p, ctypes.c_int]
        L.orc_dequant_row.restype = ctypes.c_int
        L.orc_dequant_row.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, _c_f32p]
        L.orc_dot_fn_for.restype = ctypes.c_void_p
        L.orc_dot_fn_for.argtypes = [ctypes.c_int]
        L.orc_simd_dot_fn_for.restype = ctypes.c_void_p
        L.orc_simd_dot_fn_for.argtypes = [ctypes.c_int]
        L.orc_simd_tier.restype = ctypes.c_char_p
        L.orc_simd_tier.argtypes = [ctypes.c_int]
        L.orc_simd_dot_q8_0_avx2.restype = ctypes.c_void_p
        L.orc_simd_dot_q8_0_avx2.argtypes = []
        L.orc_quant_fn_for.restype = ctypes.c_void_p
        L.orc_quant_fn_for.argtypes = [ctypes.c_int]
        for name in ("orc_iq3xxs_grid", "orc_iq3s_grid"):
            getattr(L, name).restype = ctypes.c_uint32
            getattr(L, name).argtypes = [ctypes.c_int]
        L.orc_ksigns.restype = ctypes.c_uint8
        L.orc_ksigns.argtypes = [ctypes.c_int]

    def f16_to_f32(self, h: int) -> float:
        return self.lib.orc_f16_to_f32(h)

    def f32_to_f16(self, x: float) -> int:
        return self.lib.orc_f32_to_f16(x)

    def quantize_act(self, ttype: int, x: np.ndarray) -> np.ndarray:
        """x: [k, cols] or [cols] f32 -> [k, act_bytes] uint8 (reference layout)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        x2 = x.reshape(-1, x.shape[-1])
        cols = x2.shape[1]
        out = np.zeros((x2.shape[0], act_bytes(ttype, cols)), np.uint8)
        for t in range(x2.shape[0]):
            rc = self.lib.orc_quantize_act(ttype, cols, _ptr(x2[t], _c_f32p), _ptr(out[t], _c_u8p))
            assert rc == 0
        return out.reshape(x.shape[:-1] + (out.shape[1],))

    def dot(self, ttype: int, wrow: np.ndarray, arow: np.ndarray, cols: int) -> float:
        return self.lib.orc_dot(ttype, cols, _ptr(wrow), _ptr(arow))

    def block_ints(self, ttype: int, W: np.ndarray, act: np.ndarray, cols: int) -> np.ndarray:
        """Per-block integers for every (token, row): [k, rows, nints]."""
        W = np.ascontiguousarray(W).reshape(-1, row_bytes(ttype, cols))
        act = np.ascontiguousarray(act).reshape(-1, act_bytes(ttype, cols))
        nb = cols // GEOM[ttype][0]
        ni = NINTS.get(ttype, 1) * nb
        out = np.zeros((act.shape[0], W.shape[0], ni), np.int32)
        for t in range(act.shape[0]):
            for r in range(W.shape[0]):
                n = self.lib.orc_row_block_ints(ttype, cols, _ptr(W[r]), _ptr(act[t]),
                                                _ptr(out[t, r], _c_i32p))
                assert n == ni
        return out

    def matvec(self, ttype: int, W: np.ndarray, x: np.ndarray, nthreads: int = 1) -> np.ndarray:
        """x: [k, cols] f32 -> out [k, rows] (out[t, r] = W[r] . x_t)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        x2 = x.reshape(-1, x.shape[-1])
        k, cols = x2.shape
        W = np.ascontiguousarray(W).reshape(-1, row_bytes(ttype, cols))
        rows = W.shape[0]
        out = np.zeros((k, rows), np.float32)
        rc = self.lib.orc_matvec_batch(ttype, rows, cols, k, _ptr(W), _ptr(x2, _c_f32p),
                                       _ptr(out, _c_f32p), nthreads)
        assert rc == 0
        return out.reshape(x.shape[:-1] + (rows,))

    def matvec_q_fn(self, dot_fn_addr: int, ttype: int, W: np.ndarray, act: np.ndarray,
                    cols: int, out: np.ndarray, nthreads: int) -> None:
        """Dot phase only, over a caller-chosen row-dot function address."""
        act = np.ascontiguousarray(act).reshape(-1, act_bytes(ttype, cols))
        rows = out.shape[-1]
        rc = self.lib.orc_matvec_q_fn(dot_fn_addr, ttype, rows, cols, act.shape[0], _ptr(W),
                                      _ptr(act), _ptr(out, _c_f32p), nthreads)
        assert rc == 0

    def dequant_row(self, ttype: int, wrow: np.ndarray, cols: int) -> np.ndarray:
        out = np.zeros(cols, np.float32)
        assert self.lib.orc_dequant_row(ttype, cols, _ptr(np.ascontiguousarray(wrow)),
                                        _ptr(out, _c_f32p)) == 0
        return out

    def dot_fn_addr(self, ttype: int) -> int:
        return self.lib.orc_dot_fn_for(ttype)

    def simd_dot_fn_addr(self, ttype: int) -> int:
        """The row dot at this host's ISA tier (oracle_simd.c)."""
        return self.lib.orc_simd_dot_fn_for(ttype)

    def simd_tier(self, ttype: int) -> str:
        return self.lib.orc_simd_tier(ttype).decode()

    def simd_q8_0_avx2_addr(self) -> int:
        return self.lib.orc_simd_dot_q8_0_avx2() or 0

    def matvec_dot(self, dot_fn_addr: int, ttype: int, W: np.ndarray, x: np.ndarray,
                   nthreads: int = 1) -> np.ndarray:
        """matvec with a chosen row-dot function (quantize with the oracle, then dot)."""
        x2 = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, x.shape[-1])
        cols = x2.shape[1]
        act = self.quantize_act(ttype, x2)
        W = np.ascontiguousarray(W).reshape(-1, row_bytes(ttype, cols))
        out = np.zeros((x2.shape[0], W.shape[0]), np.float32)
        self.matvec_q_fn(dot_fn_addr, ttype, W, act, cols, out, nthreads)
        return out

    def iq3_grid(self, ttype: int) -> np.ndarray:
        """The oracle's IQ3_XXS (256) or IQ3_S (512) grid as u32 entries."""
        n, f = (256, self.lib.orc_iq3xxs_grid) if ttype == TT_IQ3_XXS else (512, self.lib.orc_iq3s_grid)
        return np.array([f(i) for i in range(n)], np.uint32)

    def ksigns(self) -> np.ndarray:
        return np.array([self.lib.orc_ksigns(i) for i in range(128)], np.uint8)


class RefKernels:
    """The reference's own x86 kernels, compiled from its sources into oracle/_ref."""

    DOTS = {TT_Q8_0: "q8_0_q8_0", TT_Q4_K: "q4_k_q8_k", TT_Q6_K: "q6_k_q8_k", TT_Q5_K: "q5_k_q8_k",
            TT_Q3_K: "q3_k_q8_k", TT_Q2_K: "q2_k_q8_k", TT_Q4_0: "q4_0_q8_0", TT_Q4_1: "q4_1_q8_0"}
    QUANTS = {32: "quantize_q8_0", 256: "quantize_q8_K"}

    def __init__(self, path: Path = REF_SO):
        if not path.exists():
            raise FileNotFoundError(path)
        L = self.lib = ctypes.CDLL(str(path))
        for name in list(self.DOTS.values()) + ["k512_q8_0_q8_0_vnni"]:
            f = getattr(L, name)
            f.restype = ctypes.c_float
            f.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
        for name in self.QUANTS.values():
            f = getattr(L, name)
            f.restype = None
            f.argtypes = [ctypes.c_int, _c_f32p, _c_u8p]
        L.cpu_get_features_string.restype = ctypes.c_char_p
        L.cpu_has_avx512_vnni.restype = ctypes.c_int
        L.cpu_has_avx2.restype = ctypes.c_int

    def features(self) -> str:
        s = self.lib.cpu_get_features_string()
        return s.decode() if s else ""

    def tier(self) -> str:
        if self.lib.cpu_has_avx512_vnni():
            return "avx512vnni(q8_0)+avx2(k-quants)"
        return "avx2" if self.lib.cpu_has_avx2() else "scalar"

    def has_dot(self, ttype: int) -> bool:
        return ttype in self.DOTS

    def quantize_act(self, ttype: int, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        x2 = x.reshape(-1, x.shape[-1])
        cols = x2.shape[1]
        out = np.zeros((x2.shape[0], act_bytes(ttype, cols)), np.uint8)
        f = getattr(self.lib, self.QUANTS[act_block_elems(ttype)])
        for t in range(x2.shape[0]):
            f(cols, _ptr(x2[t], _c_f32p), _ptr(out[t], _c_u8p))
        return out.reshape(x.shape[:-1] + (out.shape[1],))

    def dot(self, ttype: int, wrow: np.ndarray, arow: np.ndarray, cols: int) -> float:
        return getattr(self.lib, self.DOTS[ttype])(cols, _ptr(wrow), _ptr(arow))

    def dot_fn_addr(self, ttype: int) -> int:
        return ctypes.cast(getattr(self.lib, self.DOTS[ttype]), ctypes.c_void_p).value


def load_ref() -> RefKernels | None:
    try:
        return RefKernels()
    except (FileNotFoundError, OSError):
        return None


def host_threads() -> int:
    """Host cores this process may use (affinity-aware), capped by OMP_NUM_THREADS."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)
