"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each check is chosen so a plausible restatement mistake (wrong nibble order,
dropped min term, wrong sign, off-by-one group, wrong rounding) fails it:
  * golden vectors written by the reference's own compiled kernels
    (tests/golden/ref_vectors.npz, see gen_golden.py), including unit-scale
    rows whose float result IS the exact block integer;
  * the reference test fixtures testdata/udtest (dequant(row) . A_x);
  * library routines / closed forms (numpy float16 conversion, exhaustive);
  * an exact identity for IQ4_NL: an IQ4_NL block equals a Q8_0 block holding
    the codebook values, so the reference's own q8_0_q8_0 pins it.
"""
from pathlib import Path

import numpy as np
import pytest

import pyoracle as po

GOLD = Path(__file__).resolve().parent / "golden"
IQ4NL = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113],
                 np.int8)  # reference src/iq_tables.zig:429-432


@pytest.fixture(scope="module")
def gv():
    return dict(np.load(GOLD / "ref_vectors.npz"))


# ---- f16 conversions ---------------------------------------------------------

def test_f16_decode_exhaustive(oracle):
    codes = np.arange(65536, dtype=np.uint16)
    want = codes.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(c)) for c in codes], np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32) & 0x7FFFFFFF, want[fin].view(np.uint32) & 0x7FFFFFFF)
    assert np.array_equal(np.signbit(got[fin & (want != 0)]), np.signbit(want[fin & (want != 0)]))
    assert np.all(np.isinf(got[np.isinf(want)]))
    assert np.all(np.isnan(got[np.isnan(want)]))


def test_f16_encode_matches_round_to_nearest_even(oracle):
    rng = np.random.default_rng(3)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.uniform(-9, 5, 20000).astype(np.float32),
        (np.arange(-70000, 70000, 7, dtype=np.float32)),
        np.float32([0.0, -0.0, 65504.0, 65519.0, 65520.0, 6e-8, 2.98e-8, 5.96e-8, 1e-40]),
    ]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16(float(v)) for v in x], np.uint16)
    # documented reference quirk: values rounding up out of the subnormal range
    quirk = (np.abs(x) >= np.float32(1023.5 * 2.0 ** -24)) & (np.abs(x) < np.float32(2.0 ** -14))
    assert np.array_equal(got[~quirk], want[~quirk])
    assert np.all(got[quirk] & 0x7FFF == 0x0380)


def test_f16_encode_nan_maps_to_inf(oracle):
    assert oracle.f32_to_f16(float("nan")) & 0x7FFF == 0x7C00
    assert oracle.f32_to_f16(float("inf")) == 0x7C00
    assert oracle.f32_to_f16(float("-inf")) == 0xFC00


# ---- quantizers against the reference's compiled output ----------------------

@pytest.mark.parametrize("name,tt", [("q8_0", po.TT_Q8_0), ("q8_k", po.TT_Q4_K)])
def test_quantizer_golden(oracle, gv, name, tt):
    got = oracle.quantize_act(tt, gv[f"quant_{name}_x"])
    assert np.array_equal(got, gv[f"quant_{name}_act"])


def test_quantizer_q8_0_quirk_row_present(gv):
    # the golden set really exercises the 0x0380 header (kernels32.c:96)
    q = gv["quant_q8_0_act"]
    act = q.reshape(q.shape[0], -1, 34)
    heads = act[:, :, 0].astype(np.uint16) | (act[:, :, 1].astype(np.uint16) << 8)
    assert np.any(heads == 0x0380)


@pytest.mark.parametrize("tt", [po.TT_Q8_0, po.TT_Q4_K])
def test_quantizer_vs_ref_random(oracle, ref, tt):
    rng = np.random.default_rng(99)
    x = (rng.standard_normal((64, 1024)) * 10.0 ** rng.uniform(-6, 4, (64, 1))).astype(np.float32)
    x[3, 5] = np.nan
    x[4, 7] = np.inf
    x[5, :] = -0.0
    assert np.array_equal(oracle.quantize_act(tt, x), ref.quantize_act(tt, x))


def test_q8_k_bsums_and_clamp(oracle):
    x = np.linspace(-3, 3, 512).astype(np.float32)
    a = oracle.quantize_act(po.TT_Q4_K, x).reshape(2, 292)
    for b in range(2):
        qs = a[b, 4:260].view(np.int8).astype(np.int32)
        bs = a[b, 260:292].view(np.int16)
        assert np.array_equal(bs, qs.reshape(16, 16).sum(1))
        assert qs.min() >= -127 and qs.max() <= 127


# ---- block integers pinned bit for bit by unit-scale reference rows ---------

@pytest.mark.parametrize("name,tt,key", [("q8_0", po.TT_Q8_0, "isum"), ("q4_k", po.TT_Q4_K, "isum"),
                                         ("q4_k", po.TT_Q4_K, "summs"), ("q6_k", po.TT_Q6_K, "isum"),
                                         ("q5_k", po.TT_Q5_K, "isum"), ("q5_k", po.TT_Q5_K, "summs"),
                                         ("q3_k", po.TT_Q3_K, "isum"), ("q2_k", po.TT_Q2_K, "isum"),
                                         ("q2_k", po.TT_Q2_K, "summs"), ("q4_0", po.TT_Q4_0, "isum"),
                                         ("q4_1", po.TT_Q4_1, "isum"), ("q4_1", po.TT_Q4_1, "summs")])
def test_block_ints_unit_scale(oracle, gv, name, tt, key):
    w, a, val = gv[f"{name}_unit_{key}_w"], gv[f"{name}_unit_{key}_a"], gv[f"{name}_unit_{key}_val"]
    be = po.GEOM[tt][0]
    got = np.array([oracle.block_ints(tt, w[i:i + 1], a[i:i + 1], be)[0, 0] for i in range(len(w))])
    if po.NINTS.get(tt, 1) == 2:
        # the K-quant mins term is subtracted (dmin * summs), the Q4_1 one added (m * sumy)
        sign = 1 if tt == po.TT_Q4_1 else -1
        got = got[:, 0] if key == "isum" else sign * got[:, 1]
    else:
        got = got[:, 0]
    assert np.all(np.abs(val) < 2 ** 24)  # exactly representable
    assert np.array_equal(got.astype(np.float32), val)


@pytest.mark.parametrize("name,tt", [("q8_0", po.TT_Q8_0), ("q4_k", po.TT_Q4_K), ("q6_k", po.TT_Q6_K),
                                     ("q5_k", po.TT_Q5_K), ("q3_k", po.TT_Q3_K), ("q2_k", po.TT_Q2_K),
                                     ("q4_0", po.TT_Q4_0), ("q4_1", po.TT_Q4_1)])
def test_row_dot_golden(oracle, gv, name, tt):
    w, x, want = gv[f"{name}_w"], gv[f"{name}_x"], gv[f"{name}_dot"]
    cols = x.shape[1]
    got = oracle.matvec(tt, w, x)
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel < 1e-6, rel
    if tt == po.TT_Q8_0:  # same sequential fold as the VNNI tier
        assert np.array_equal(got, want)
    assert cols % 256 == 0


@pytest.mark.parametrize("tt", [po.TT_Q8_0, po.TT_Q4_K, po.TT_Q6_K, po.TT_Q5_K, po.TT_Q3_K, po.TT_Q2_K,
                                po.TT_Q4_0, po.TT_Q4_1])
def test_row_dot_vs_ref_random(oracle, ref, tt):
    from qwen35_amd import synth
    cols = 2560 if tt != po.TT_Q6_K else 2816
    w = synth.make_weight(tt, 64, cols, seed=5, tag=tt)
    x = synth.make_act(cols, 2, seed=5)
    act = ref.quantize_act(tt, x)
    want = np.array([[ref.dot(tt, w[r], act[t], cols) for r in range(64)] for t in range(2)])
    got = oracle.matvec(tt, w, x)
    assert np.linalg.norm(got - want) / np.linalg.norm(want) < 1e-6


def _iq4nl_as_q8_0(wrow: np.ndarray, cols: int) -> np.ndarray:
    blk = wrow.reshape(cols // 32, 18)
    out = np.zeros((cols // 32, 34), np.uint8)
    out[:, 0:2] = blk[:, 0:2]
    lo, hi = blk[:, 2:] & 15, blk[:, 2:] >> 4
    out[:, 2:18] = IQ4NL[lo].view(np.uint8)
    out[:, 18:34] = IQ4NL[hi].view(np.uint8)
    return out.reshape(-1)


def test_iq4_nl_equals_q8_0_of_codebook(oracle, ref):
    from qwen35_amd import synth
    cols = 2560
    w = synth.make_weight(po.TT_IQ4_NL, 48, cols, seed=9, tag=20)
    x = synth.make_act(cols, 2, seed=9)
    act = ref.quantize_act(po.TT_Q8_0, x)
    got = oracle.matvec(po.TT_IQ4_NL, w, x)
    for t in range(2):
        want = np.array([ref.dot(po.TT_Q8_0, _iq4nl_as_q8_0(w[r], cols), act[t], cols)
                         for r in range(48)], np.float32)
        assert np.array_equal(got[t], want)  # same integers, same sequential fold
    ints = oracle.block_ints(po.TT_IQ4_NL, w, act, cols)
    w8 = np.stack([_iq4nl_as_q8_0(w[r], cols) for r in range(48)])
    ints8 = oracle.block_ints(po.TT_Q8_0, w8, act, cols)
    assert np.array_equal(ints, ints8)


def _iq4xs_as_iq4nl(wrow: np.ndarray, cols: int) -> tuple[np.ndarray, np.ndarray]:
    """IQ4_XS super-blocks -> IQ4_NL blocks with the same indices, and the
    6-bit scales ls - 32 of each 32-value block (iq_kernels.c:976-979)."""
    blk = wrow.reshape(cols // 256, 136)
    nl = np.zeros((cols // 256, 8, 18), np.uint8)
    nl[:, :, 2:] = blk[:, 8:].reshape(-1, 8, 16)
    sh = blk[:, 2].astype(np.int64) | (blk[:, 3].astype(np.int64) << 8)
    ls = np.zeros((cols // 256, 8), np.int64)
    for ib in range(8):
        ls[:, ib] = ((blk[:, 4 + ib // 2] >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4)
    return nl.reshape(-1), (ls - 32).reshape(-1)


def test_iq4_xs_block_ints_equal_iq4_nl(oracle):
    """IQ4_XS uses the IQ4_NL codebook with one index per value: with the same
    int8 activation values its 32-value block integers ARE the IQ4_NL block
    integers of the re-packed indices (pinned above by the reference's
    q8_0_q8_0), and its row dot is sum_b (d*dy*(ls_b - 32)) * int_b."""
    from qwen35_amd import synth
    cols, rows = 1024, 16
    w = synth.make_weight(po.TT_IQ4_XS, rows, cols, seed=8, tag=23)
    # integer activations with +-127 in every 32-block: Q8_K and Q8_0 both
    # quantize them to themselves with scale 1
    rng = np.random.default_rng(8)
    x = rng.integers(-127, 128, (2, cols)).astype(np.float32)
    x[:, ::32] = 127.0
    a_k = oracle.quantize_act(po.TT_IQ4_XS, x)
    a_0 = oracle.quantize_act(po.TT_IQ4_NL, x)
    assert np.all(a_k[:, 0:4].view(np.float32) == 1.0)
    ints_xs = oracle.block_ints(po.TT_IQ4_XS, w, a_k, cols)
    nl = np.stack([_iq4xs_as_iq4nl(w[r], cols)[0] for r in range(rows)])
    ints_nl = oracle.block_ints(po.TT_IQ4_NL, nl, a_0, cols)
    assert np.array_equal(ints_xs, ints_nl)
    # the float fold against the unpacked scales
    d = w.reshape(rows, cols // 256, 136)[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float32)
    got = oracle.matvec(po.TT_IQ4_XS, w, x)
    for r in range(rows):
        ls = _iq4xs_as_iq4nl(w[r], cols)[1]
        want = np.sum(np.repeat(d[r], 8).astype(np.float64) * ls * ints_xs[:, r, :], axis=1)
        assert np.allclose(got[:, r], want, rtol=1e-5, atol=1e-6 * np.abs(want).max())


# ---- the reference's own fixtures (testdata/udtest) ------------------------------

UD = {po.TT_Q8_0: ("Q8_0", 320), po.TT_Q4_K: ("Q4_K", 144), po.TT_Q6_K: ("Q6_K", 210),
      po.TT_IQ4_NL: ("IQ4_NL", 144), po.TT_Q5_K: ("Q5_K", 176), po.TT_Q3_K: ("Q3_K", 110),
      po.TT_IQ4_XS: ("IQ4_XS", 136), po.TT_Q4_0: ("Q4_0", 144), po.TT_Q4_1: ("Q4_1", 160),
      po.TT_IQ3_XXS: ("IQ3_XXS", 98), po.TT_IQ3_S: ("IQ3_S", 110)}


def _udtest(tt):
    name, stride = UD[tt]
    raw = np.fromfile(GOLD / "udtest" / f"{name}.bin", np.uint8).reshape(-1, stride)
    exp = np.fromfile(GOLD / "udtest" / f"{name}_expected.f32", np.float32)
    ax = np.fromfile(GOLD / "udtest" / "A_x.f32", np.float32)
    return raw[:, :po.row_bytes(tt, 256)], exp, ax


@pytest.mark.parametrize("tt", list(UD))
def test_udtest_fixture_bit_exact(oracle, tt):
    """The fixture's expected values are dequant(row) . A_x folded in f32 one
    value at a time (product, then sum: quant_dequant.zig:1155-1161).  The
    oracle's dequant reproduces every one of them bit for bit, so every
    dequantized value that a fixture row holds is pinned."""
    rows, exp, ax = _udtest(tt)
    deq = np.stack([oracle.dequant_row(tt, rows[r], 256) for r in range(len(rows))])
    acc = np.zeros(len(rows), np.float32)
    for i in range(256):
        acc = acc + deq[:, i] * ax[i]  # float32 product, then float32 sum
    assert acc.dtype == np.float32
    assert np.array_equal(acc, exp)


@pytest.mark.parametrize("tt", list(UD))
def test_udtest_dequant_fixture(oracle, tt):
    name, stride = UD[tt]
    raw = np.fromfile(GOLD / "udtest" / f"{name}.bin", np.uint8).reshape(-1, stride)
    exp = np.fromfile(GOLD / "udtest" / f"{name}_expected.f32", np.float32)
    ax = np.fromfile(GOLD / "udtest" / "A_x.f32", np.float32)
    rb = po.row_bytes(tt, 256)
    rows = raw[:, :rb]  # Q8_0 rows carry 48 bytes of padding after 8 blocks
    deq = np.stack([oracle.dequant_row(tt, rows[r], 256) for r in range(len(rows))])
    err = np.abs(deq.astype(np.float64) @ ax - exp)
    assert err.max() < 1e-3, err.max()  # quant_dequant.zig:1175-1205 bound
    # the quantized-activation row dot against the dequantized row times the
    # exact f32 view of the quantized activation (simd_tests256.zig:120-159,
    # whose SIMD tiers are held to 5e-3; the oracle's exact integers to 1e-5)
    act = oracle.quantize_act(tt, ax[None, :])[0]
    if po.act_block_elems(tt) == 32:
        blk = act.reshape(-1, 34)
        xq = (blk[:, 0:2].copy().view(np.float16).astype(np.float64) * blk[:, 2:].view(np.int8)).reshape(-1)
    else:
        xq = np.float64(act[0:4].view(np.float32)[0]) * act[4:260].view(np.int8)
    want = deq.astype(np.float64) @ xq
    got = oracle.matvec(tt, np.ascontiguousarray(rows), ax[None, :])[0]
    rel = np.abs(got - want) / np.maximum(np.abs(want), 1.0)
    assert rel.max() < 1e-5, rel.max()


def test_hand_computed_q8_0_block(oracle):
    # backend_cpu.zig:1366-1379: d = 1.5, q = {0, 1, -1, 32, -128}
    blk = np.zeros(34, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.5).tobytes(), np.uint8)
    blk[2:7] = np.array([0, 1, -1, 32, -128], np.int8).view(np.uint8)
    deq = oracle.dequant_row(po.TT_Q8_0, blk, 32)
    assert list(deq[:5]) == [0.0, 1.5, -1.5, 48.0, -192.0]


# ---- driver semantics ---------------------------------------------------------------

@pytest.mark.parametrize("tt", [po.TT_Q8_0, po.TT_Q4_K, po.TT_Q6_K, po.TT_IQ4_NL])
def test_threads_and_batch_bit_identical(oracle, tt):
    from qwen35_amd import synth
    cols = 1024
    w = synth.make_weight(tt, 300, cols, seed=2, tag=tt)
    x = synth.make_act(cols, 3, seed=2)
    one = oracle.matvec(tt, w, x, nthreads=1)
    many = oracle.matvec(tt, w, x, nthreads=4)
    assert np.array_equal(one, many)
    for t in range(3):
        assert np.array_equal(oracle.matvec(tt, w, x[t:t + 1], nthreads=1)[0], one[t])


def test_zero_activation_gives_zero(oracle):
    from qwen35_amd import synth
    w = synth.make_weight(po.TT_Q4_K, 8, 512, seed=1)
    out = oracle.matvec(po.TT_Q4_K, w, np.zeros((1, 512), np.float32))
    assert np.all(out == 0)


@pytest.mark.parametrize("tt", [po.TT_Q8_0, po.TT_IQ4_NL, po.TT_Q4_K, po.TT_Q6_K])
def test_dequant_signed_zero_scale(oracle, tt):
    """The reference dequant converts the f16 scale with @floatCast
    (quant_dequant.zig:34-37), which keeps -0: d * q then carries the IEEE sign
    of the product.  Closed form with numpy's exact float16 conversion."""
    be, bb = po.GEOM[tt]
    cols = be
    w = np.zeros(bb, np.uint8)
    rng = np.random.default_rng(0)
    w[:] = rng.integers(0, 256, bb)
    off = 208 if tt == po.TT_Q6_K else 0
    w[off:off + 2] = [0x00, 0x80]  # -0
    if tt == po.TT_Q4_K:
        w[2:4] = [0x00, 0x80]
    out = oracle.dequant_row(tt, w, cols)
    assert np.all(out == 0)
    d = np.float32(np.float16(-0.0))
    assert np.signbit(d)
    if tt == po.TT_Q8_0:
        q = w[2:].view(np.int8).astype(np.float32)
        assert np.array_equal(np.signbit(out), np.signbit(d * q))
    elif tt == po.TT_IQ4_NL:
        idx = np.concatenate([w[2:18] & 15, w[2:18] >> 4])
        q = IQ4NL[idx].astype(np.float32)
        assert np.array_equal(np.signbit(out), np.signbit(d * q))


# ---- IQ3_XXS / IQ3_S grids and signs ------------------------------------------------

def _iq3_uses(tt, rows):
    """(row, value position, grid entry, byte j) for every value of the rows,
    decoded from the index stream (iq_kernels.c:612-643, :1728-1772)."""
    out = []
    for r, row in enumerate(rows):
        for ib in range(8):
            for k in range(8):  # 4-value group k of the 32-value sub-block
                e = int(row[2 + 8 * ib + k])
                if tt == po.TT_IQ3_S:
                    e |= ((int(row[66 + ib]) >> k) & 1) << 8
                for j in range(4):
                    out.append((r, 32 * ib + 4 * k + j, e, j))
    return out


def test_ksigns_even_parity(oracle):
    # ksigns_iq2xs (iq_tables.zig:42-61): the low 7 bits are the index, bit 7
    # makes the number of negated values even
    ks = oracle.ksigns()
    assert np.array_equal(ks & 127, np.arange(128))
    assert all(bin(int(v)).count("1") % 2 == 0 for v in ks)


@pytest.mark.parametrize("tt", [po.TT_IQ3_XXS, po.TT_IQ3_S])
def test_iq3_grid_levels_and_order(oracle, tt):
    g = oracle.iq3_grid(tt)
    levels = [4, 12, 20, 28, 36, 44, 52, 62] if tt == po.TT_IQ3_XXS else list(range(1, 16, 2))
    assert np.all(np.isin(g.view(np.uint8), levels))
    assert np.all(np.diff(g.astype(np.int64)) > 0)  # strictly increasing as u32
    assert g[0] == (0x04040404 if tt == po.TT_IQ3_XXS else 0x01010101)


@pytest.mark.parametrize("tt", [po.TT_IQ3_XXS, po.TT_IQ3_S])
def test_iq3_fixture_pins_grid_entries(oracle, tt):
    """Every grid entry a fixture row uses is pinned by the bit-exact fixture
    test: the oracle's dequant of that value is +-db * byte j of the entry,
    checked here against the decoded index stream, and any other byte would
    move the row's f32 result.  IQ3_XXS rows use all 256 entries and all 128
    sign indices; IQ3_S rows use 501 of its 512 entries."""
    rows, _, _ = _udtest(tt)
    g = oracle.iq3_grid(tt).view(np.uint8).reshape(-1, 4)
    deq = np.stack([oracle.dequant_row(tt, rows[r], 256) for r in range(len(rows))])
    d = rows[:, 0:2].copy().view(np.float16)[:, 0].astype(np.float32)
    used = set()
    for r, pos, e, j in _iq3_uses(tt, rows):
        ib = pos // 32
        if tt == po.TT_IQ3_XXS:
            ls = int(rows[r, 66 + 4 * ib + 3]) >> 4
            db = d[r] * (np.float32(0.5) + np.float32(ls)) * np.float32(0.5)
        else:
            db = d[r] * np.float32(2 * ((int(rows[r, 106 + ib // 2]) >> (4 * (ib % 2))) & 15) + 1)
        assert abs(deq[r, pos]) == np.float32(db * np.float32(g[e, j])), (r, pos, e, j)
        used.add(e)
    if tt == po.TT_IQ3_XXS:
        assert len(used) == 256
        signs = {(int(rows[r, 66 + 4 * ib:70 + 4 * ib].view(np.uint32)[0]) >> (7 * l)) & 127
                 for r in range(len(rows)) for ib in range(8) for l in range(4)}
        assert len(signs) == 128
    else:
        # the 11 entries no fixture row uses are pinned by the table fixture
        # (test_iq3_grid_equals_reference_table)
        assert len(used) == 501
        assert sorted(set(range(512)) - used) == [32, 57, 71, 100, 104, 113, 197, 200, 207, 216, 491]


@pytest.mark.parametrize("tt", [po.TT_IQ3_XXS, po.TT_IQ3_S])
def test_iq3_grid_equals_reference_table(oracle, tt):
    """Every entry of the oracle's grid (built from the product's own
    encoding in qwen35_amd/csrc/iq_grids.h) equals the reference's table
    (src/iq_tables.zig:322-355 iq3xxs_grid, :360-425 iq3s_grid), read as
    numbers into tests/golden/iq3_grids.npz by tests/golden/gen_iq3_grids.py.
    This pins the 11 IQ3_S entries no udtest fixture row uses."""
    fix = np.load(GOLD / "iq3_grids.npz")
    want = fix["iq3xxs_grid"] if tt == po.TT_IQ3_XXS else fix["iq3s_grid"]
    got = oracle.iq3_grid(tt)
    assert want.shape == got.shape
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, [(int(i), hex(int(got[i])), hex(int(want[i]))) for i in bad[:8]]


@pytest.mark.parametrize("tt", [po.TT_IQ3_XXS, po.TT_IQ3_S])
def test_iq3_dot_equals_scaled_dequant(oracle, tt):
    """With integer activations whose Q8_K scale is exactly 1, the row dot is
    sum_b d_b * sum_ib (2 ls + 1) * sumi_ib (times 1/4 for IQ3_XXS): the exact
    integers of block_ints against the dequantized values (a closed form: for
    every value, dequant = d * (2 ls + 1) / 4 (or 1) * signed grid value)."""
    from qwen35_amd import synth
    cols, nrows = 1024, 12
    w = synth.make_weight(tt, nrows, cols, seed=4, tag=tt)
    rng = np.random.default_rng(4)
    x = rng.integers(-127, 128, (2, cols)).astype(np.float32)
    x[:, ::256] = 127.0
    act = oracle.quantize_act(tt, x)
    assert np.all(act[:, 0:4].view(np.float32) == 1.0)
    ints = oracle.block_ints(tt, w, act, cols)  # [tokens][rows][cols/32]
    for r in range(nrows):
        deq = oracle.dequant_row(tt, w[r], cols).astype(np.float64)
        blk = w[r].reshape(cols // 256, -1)
        d = blk[:, 0:2].copy().view(np.float16)[:, 0].astype(np.float64)
        if tt == po.TT_IQ3_XXS:
            ls = np.stack([blk[:, 66 + 4 * ib + 3] >> 4 for ib in range(8)], 1).reshape(-1)
            scale = np.repeat(d, 8) * (2 * ls + 1) / 4.0
        else:
            ls = np.stack([(blk[:, 106 + ib // 2] >> (4 * (ib % 2))) & 15 for ib in range(8)], 1).reshape(-1)
            scale = np.repeat(d, 8) * (2 * ls + 1)
        # the signed grid values times q8, per 32-value block, from the dequant
        gq = np.round(deq / np.repeat(scale, 32)).reshape(-1, 32)
        for t in range(2):
            assert np.array_equal((gq * x[t].reshape(-1, 32)).sum(1), ints[t, r])
        got = oracle.matvec(tt, w[r:r + 1], x)[:, 0]
        want = ints[:, r, :].astype(np.float64) @ scale
        assert np.allclose(got, want, rtol=2e-6, atol=0)


def test_q2_k_dequant_equals_block_ints(oracle):
    """Ties the Q2_K dequant (quant_dequant.zig:892-919) to the block integers
    pinned bit for bit against the reference build (kernels256.c:232-257):
    each value dequantizes to d * (scales[g] & 15) * q - dmin * (scales[g] >> 4),
    so with d = 1, dmin = 0 the dequantized row dotted with integer activations
    (Q8_K scale exactly 1) is isum, and with d = 0, dmin = 1 it is -summs.  A
    value read from the wrong byte, shift or 16-value group, a scale nibble
    swapped, or the mins term's sign flipped moves one of the two sums; with
    d = 2^-3, dmin = 2^-5 both terms come back exactly."""
    rng = np.random.default_rng(11)
    cols, nrows = 1024, 6
    nb = cols // 256
    w = rng.integers(0, 256, (nrows, nb, 84), dtype=np.uint8)
    x = rng.integers(-127, 128, (3, cols)).astype(np.float32)
    x[:, ::256] = 127.0
    act = oracle.quantize_act(po.TT_Q2_K, x)
    for b in range(nb):
        assert act[0, 292 * b:292 * b + 4].view(np.float32)[0] == 1.0
    h = {v: np.array([v], np.float16).view(np.uint8) for v in (0.0, 1.0, 0.125, 0.03125)}
    for d, dmin in ((1.0, 0.0), (0.0, 1.0), (0.125, 0.03125)):
        w[:, :, 80:82] = h[d]
        w[:, :, 82:84] = h[dmin]
        rows = w.reshape(nrows, -1)
        ints = oracle.block_ints(po.TT_Q2_K, rows, act, cols).reshape(3, nrows, nb, 2).astype(np.float64)
        for r in range(nrows):
            deq = oracle.dequant_row(po.TT_Q2_K, rows[r], cols).astype(np.float64).reshape(nb, 256)
            for t in range(3):
                got = (deq * x[t].reshape(nb, 256)).sum(1)
                want = d * ints[t, r, :, 0] - dmin * ints[t, r, :, 1]
                assert np.array_equal(got, want), (d, dmin, r, t)


# ---- the host-ISA tiers of the restatement (oracle_simd.c, the CPU baseline) --

SIMD_CASES = [(po.TT_IQ4_NL, 2560), (po.TT_Q8_0, 1024), (po.TT_Q4_K, 2560), (po.TT_Q6_K, 9728)]


@pytest.mark.parametrize("tt,cols", SIMD_CASES, ids=[po.NAMES[c[0]] for c in SIMD_CASES])
def test_simd_tier_matches_scalar(oracle, tt, cols):
    """Same integers on every tier; IQ4_NL (AVX2) and Q8_0 (VNNI) fold the
    blocks sequentially like the scalar restatement, so they must agree bit
    for bit; the 8-lane FMA folds (Q4_K, Q6_K, Q8_0 AVX2) within 1e-6."""
    from qwen35_amd import synth
    w = synth.make_weight(tt, 48, cols, seed=21, tag=tt)
    x = synth.make_act(cols, 3, seed=22)
    want = oracle.matvec(tt, w, x)
    got = oracle.matvec_dot(oracle.simd_dot_fn_addr(tt), tt, w, x)
    tier = oracle.simd_tier(tt)
    if tt == po.TT_IQ4_NL or tier in ("avx512vnni", "scalar"):
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), tier
    else:
        assert np.linalg.norm(got - want) / np.linalg.norm(want) < 1e-6
    if tt == po.TT_Q8_0 and oracle.simd_q8_0_avx2_addr():
        g2 = oracle.matvec_dot(oracle.simd_q8_0_avx2_addr(), tt, w, x)
        assert np.linalg.norm(g2 - want) / np.linalg.norm(want) < 1e-6


@pytest.mark.parametrize("tt", [po.TT_Q8_0, po.TT_Q4_K, po.TT_Q6_K], ids=["Q8_0", "Q4_K", "Q6_K"])
def test_simd_tier_matches_reference_build(oracle, ref, tt):
    """The restated tiers against the reference's own compiled kernels, which
    dispatch to the same tier on this host: bit-identical floats."""
    from qwen35_amd import synth
    cols = {po.TT_Q8_0: 2048, po.TT_Q4_K: 5120, po.TT_Q6_K: 9728}[tt]
    w = synth.make_weight(tt, 40, cols, seed=23, tag=tt)
    x = synth.make_act(cols, 2, seed=24)
    got = oracle.matvec_dot(oracle.simd_dot_fn_addr(tt), tt, w, x)
    want = oracle.matvec_dot(ref.dot_fn_addr(tt), tt, w, x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
