"""Write tests/golden/ref_vectors.npz from the reference's own compiled x86
kernels (oracle/_ref/libqref.so, built from /root/reference sources by
oracle/Makefile).  Run in the build container only:

    make -C oracle ref && python tests/golden/gen_golden.py

Contents (small seeded inputs and the reference's outputs on them):
  quant_q8_0_x / _act          quantize_q8_0 input rows and output bytes
  quant_q8_k_x / _act          quantize_q8_K input rows and output bytes
  <T>_w, <T>_x, <T>_dot        weight rows, activation rows (f32) and the
                               reference row dot (T = q8_0, q4_k, q6_k, q5_k,
                               q3_k, q2_k, q4_0, q4_1) of each
                               weight row against the reference-quantized row
  <T>_unit_*                   rows with unit scales (d = 1, dmin = 0 / d = 0,
                               dmin = 1; Q4_1: d = 1, m = 0 / d = 0, m = 1)
                               whose float result equals the exact integer
                               sums, pinning them bit for bit
  meta_tier                    CPU tier the reference dispatched to
"""
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "oracle"))
import pyoracle as po  # noqa: E402
from qwen35_amd import synth  # noqa: E402

TT = {"q8_0": po.TT_Q8_0, "q4_k": po.TT_Q4_K, "q6_k": po.TT_Q6_K, "q5_k": po.TT_Q5_K,
      "q3_k": po.TT_Q3_K, "q2_k": po.TT_Q2_K, "q4_0": po.TT_Q4_0, "q4_1": po.TT_Q4_1}
# byte offsets of (d, dmin) in each weight block; dmin None: no mins term
SCALE_AT = {po.TT_Q4_K: (0, 2), po.TT_Q5_K: (0, 2), po.TT_Q6_K: (208, None), po.TT_Q3_K: (108, None),
            po.TT_Q2_K: (80, 82), po.TT_Q8_0: (0, None), po.TT_Q4_0: (0, None), po.TT_Q4_1: (0, 2)}


def edge_rows(n: int) -> np.ndarray:
    """Activation rows that stress the quantizer rules (ties, zeros, tiny, huge)."""
    rows = []
    rng = np.random.default_rng(7)
    z = np.zeros(n, np.float32)
    rows.append(z)                                    # amax == 0
    t = np.tile(np.float32([127.0, 63.5, -63.5, 0.5, -0.5, 1.5, -2.5, 0.0]), n // 8)
    rows.append(t)                                    # exact .5 ties after scaling
    rows.append((rng.standard_normal(n) * 1e-30).astype(np.float32))  # subnormal scale
    rows.append((rng.standard_normal(n) * 3e4).astype(np.float32))    # big values
    s = rng.standard_normal(n).astype(np.float32)
    s[::37] = -0.0
    rows.append(s)
    # f16 header rounding out of the subnormal range (kernels32.c:96 quirk)
    w = rng.uniform(-1, 1, n).astype(np.float32) * np.float32(0.0077)
    w[::32] = np.float32(0.0077491)
    rows.append(w)
    return np.stack(rows)


def main():
    ref = po.RefKernels()
    out = {"meta_tier": np.array(ref.tier())}
    rng = np.random.default_rng(1234)
    for name, n in (("q8_0", 512), ("q8_k", 512)):
        x = np.concatenate([edge_rows(n), rng.standard_normal((10, n)).astype(np.float32)])
        tt = po.TT_Q8_0 if name == "q8_0" else po.TT_Q4_K
        out[f"quant_{name}_x"] = x
        out[f"quant_{name}_act"] = ref.quantize_act(tt, x)
    for name, tt in TT.items():
        cols = 512 if po.GEOM[tt][0] == 32 else 768
        rows = 12
        w = synth.make_weight(tt, rows, cols, seed=11, tag=tt)
        x = synth.make_act(cols, 3, seed=11)
        act = ref.quantize_act(tt, x)
        dots = np.array([[ref.dot(tt, w[r], act[t], cols) for r in range(rows)] for t in range(3)],
                        np.float32)
        out[f"{name}_w"], out[f"{name}_x"], out[f"{name}_dot"] = w, x, dots
        # unit-scale rows: one block per row so the float result is that block's integer
        be, bb = po.GEOM[tt]
        nblk = 16
        wb = synth.make_weight(tt, nblk, be, seed=13, tag=tt)
        ab = ref.quantize_act(tt, synth.make_act(be, nblk, seed=13))
        one = np.float16(1.0).view(np.uint16)
        variants = {}
        a1 = ab.copy()
        if be == 32:  # Q8_0 activation blocks: f16 scale
            a1[:, 0:2] = np.frombuffer(one.tobytes(), np.uint8)
        else:         # Q8_K activation blocks: f32 scale
            a1[:, 0:4] = np.frombuffer(np.float32(1.0).tobytes(), np.uint8)
        od, om = SCALE_AT[tt]
        wi = wb.copy(); wi[:, od:od + 2] = np.frombuffer(one.tobytes(), np.uint8)
        if om is not None:
            wi[:, om:om + 2] = 0
            wm = wb.copy(); wm[:, od:od + 2] = 0; wm[:, om:om + 2] = np.frombuffer(one.tobytes(), np.uint8)
            variants["summs"] = (wm, a1)
        variants["isum"] = (wi, a1)
        for key, (wv, av) in variants.items():
            vals = np.array([ref.dot(tt, wv[i], av[i], be) for i in range(nblk)], np.float32)
            out[f"{name}_unit_{key}_w"], out[f"{name}_unit_{key}_a"] = wv, av
            out[f"{name}_unit_{key}_val"] = vals
    path = Path(__file__).with_name("ref_vectors.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({path.stat().st_size} bytes), tier {ref.tier()}")


if __name__ == "__main__":
    main()
