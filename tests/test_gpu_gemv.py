"""GPU parity: HIP quantizers and GEMV against the CPU oracle, through the C ABI.

Bar: quantized activations and per-block integers bit-exact; float outputs
within 1e-5 relative L2 of the oracle (the tolerance BASELINE.json's
north_star states for the float result after scale application).
"""
import numpy as np
import pytest
import torch

import pyoracle as po
import qwen35_amd
from qwen35_amd import ops, synth

pytestmark = pytest.mark.gpu

TOL = 1e-5  # relative L2, float outputs
TYPES = po.ALL_TYPES


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


def to_dev(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def case_id(tt, rows, cols):
    return f"{po.NAMES[tt]}-{rows}x{cols}"


# ---- quantizers ------------------------------------------------------------------

QUANT_INPUTS = {
    "normal": lambda rng, k, n: rng.standard_normal((k, n)).astype(np.float32),
    "wide": lambda rng, k, n: (rng.standard_normal((k, n)) * 10.0 ** rng.uniform(-30, 30, (k, 1))).astype(np.float32),
    "ties": lambda rng, k, n: np.tile(np.float32([127, 63.5, -63.5, .5, -.5, 1.5, -2.5, 0]), (k, n // 8)),
    "zeros": lambda rng, k, n: np.zeros((k, n), np.float32),
}


@pytest.mark.parametrize("kind", list(QUANT_INPUTS))
@pytest.mark.parametrize("tt", [po.TT_Q8_0, po.TT_Q4_K])
def test_quantize_act_bit_exact(gpu, oracle, tt, kind):
    rng = np.random.default_rng(17)
    x = QUANT_INPUTS[kind](rng, 5, 4096)
    if kind == "wide":
        x[0, 3] = np.nan
        x[1, :7] = -0.0
        x[2, 9] = np.inf
    want = oracle.quantize_act(tt, x)
    got = ops.quantize_act(tt, to_dev(x, gpu)).cpu().numpy()
    assert np.array_equal(got, want)


def misaligned(x, gpu):
    """A device copy of x whose data pointer is 4 bytes past a 16-byte boundary."""
    buf = torch.empty(x.size + 4, dtype=torch.float32, device=gpu)
    assert buf.data_ptr() % 16 == 0
    view = buf[1:1 + x.size].view(x.shape)
    view.copy_(torch.from_numpy(np.ascontiguousarray(x)))
    assert view.data_ptr() % 16 == 4
    return view


@pytest.mark.parametrize("tt,k,cols", [(po.TT_Q8_0, 1, 256), (po.TT_Q8_0, 33, 1024), (po.TT_Q8_0, 1025, 1024),
                                       (po.TT_Q4_K, 3, 768), (po.TT_Q4_K, 7, 2560), (po.TT_Q4_K, 129, 65536)])
def test_quantize_wide_and_narrow_forms(gpu, oracle, tt, k, cols):
    """From 32768 blocks the wide quantizers run (16-byte rows, blocks
    numbered over tokens; here with a last workgroup only partly filled),
    below it and on rows off a 16-byte boundary the narrow ones: all give
    the oracle's bytes."""
    x = QUANT_INPUTS["wide"](np.random.default_rng(k + cols), k, cols)
    x[0, 1] = np.nan
    want = oracle.quantize_act(tt, x)
    assert np.array_equal(ops.quantize_act(tt, to_dev(x, gpu)).cpu().numpy(), want)
    assert np.array_equal(ops.quantize_act(tt, misaligned(x, gpu)).cpu().numpy(), want)


@pytest.mark.parametrize("tt,cols,lens", [(po.TT_Q8_0, 1024, [300, 1, 512, 230]), (po.TT_Q8_0, 512, [5, 1, 9, 3]),
                                          (po.TT_Q4_K, 512, [5, 1, 9, 3])])
def test_quantize_ragged_rows_at_any_alignment(gpu, oracle, tt, cols, lens):
    """The ragged packer reads each sequence's rows as they lie: 16-byte
    aligned sequences and one 4 bytes off, packed in one launch (the first
    case, 33376 Q8_0 blocks, in the wide form)."""
    rng = np.random.default_rng(5)
    seqs = [rng.standard_normal((n, cols)).astype(np.float32) for n in lens]
    dseqs = [to_dev(s, gpu) for s in seqs]
    dseqs[2] = misaligned(seqs[2], gpu)
    xq, _, total = ops.quantize_ragged(tt, dseqs, cols)
    want = oracle.quantize_act(tt, np.concatenate(seqs))
    assert np.array_equal(xq[:total].cpu().numpy(), want)


def test_quantize_header_quirk(gpu, oracle):
    # scale rounding out of the f16 subnormal range -> 0x0380 (kernels32.c:96)
    x = np.random.default_rng(1).uniform(-1, 1, 64).astype(np.float32) * np.float32(0.0077)
    x[0] = np.float32(0.0077491)
    want = oracle.quantize_act(po.TT_Q8_0, x[None])
    assert int(want[0, 0]) | (int(want[0, 1]) << 8) == 0x0380
    got = ops.quantize_q8_0(to_dev(x, gpu)).cpu().numpy()
    assert np.array_equal(got, want[0])


def test_quantize_single_entry_points(gpu, oracle):
    x = synth.make_act(2560, 1, seed=4)[0]
    assert np.array_equal(ops.quantize_q8_0(to_dev(x, gpu)).cpu().numpy(),
                          oracle.quantize_act(po.TT_Q8_0, x))
    assert np.array_equal(ops.quantize_q8_K(to_dev(x, gpu)).cpu().numpy(),
                          oracle.quantize_act(po.TT_Q4_K, x))


# ---- GEMV ---------------------------------------------------------------------------

SHAPES = {
    po.TT_Q8_0: [(300, 1024), (64, 192), (1, 64)],
    po.TT_IQ4_NL: [(200, 2560), (37, 256)],
    po.TT_Q4_K: [(100, 2560), (33, 256)],
    po.TT_Q6_K: [(50, 9728), (18, 256), (16, 2304)],
    po.TT_Q5_K: [(100, 2560), (33, 256)],
    po.TT_Q3_K: [(60, 2560), (18, 256), (16, 2304)],
    po.TT_Q2_K: [(70, 2560), (21, 256)],
    po.TT_IQ4_XS: [(80, 2560), (19, 256)],
    po.TT_Q4_0: [(200, 2560), (37, 256), (11, 224)],
    po.TT_Q4_1: [(150, 2560), (29, 256), (9, 224)],
    po.TT_IQ3_XXS: [(90, 2560), (21, 256), (16, 2304)],
    po.TT_IQ3_S: [(90, 2560), (21, 256), (16, 2304)],
}
CASES = [(tt, r, c) for tt in TYPES for (r, c) in SHAPES[tt]]


def setup(tt, rows, cols, k, dev, seed=0):
    w = synth.make_weight(tt, rows, cols, seed=seed, tag=tt)
    x = synth.make_act(cols, k, seed=seed)
    return w, x, to_dev(w, dev), to_dev(x, dev)


@pytest.mark.parametrize("tt,rows,cols", CASES, ids=[case_id(*c) for c in CASES])
def test_block_ints_bit_exact(gpu, oracle, tt, rows, cols):
    w, x, wd, xd = setup(tt, rows, cols, 2, gpu)
    act = oracle.quantize_act(tt, x)
    xq = ops.quantize_act(tt, xd)
    assert np.array_equal(xq.cpu().numpy(), act)
    if cols % (64 if po.GEOM[tt][0] == 32 else 256) or rows * po.row_bytes(tt, cols) % 4:
        # the export walks whole per-lane chunks of a dword-sized weight
        # buffer; other widths and sizes are refused
        with pytest.raises(qwen35_amd.QhipError):
            ops.block_ints(tt, wd, xq, rows, cols, 2)
        return
    got = ops.block_ints(tt, wd, xq, rows, cols, 2).cpu().numpy()
    want = oracle.block_ints(tt, w, act, cols)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("tokens", [1, 3, 8, 9])
@pytest.mark.parametrize("tt,rows,cols", CASES, ids=[case_id(*c) for c in CASES])
def test_gemv_matches_oracle(gpu, oracle, tt, rows, cols, tokens):
    w, x, wd, xd = setup(tt, rows, cols, tokens, gpu, seed=tokens)
    want = oracle.matvec(tt, w, x)
    xq = ops.quantize_act(tt, xd)
    for path in (0, 1, 3):  # auto, gemv, generic
        got = ops.mul_mat(tt, wd, xq, rows, cols, tokens, path=path).cpu().numpy()
        assert rel_l2(got, want) < TOL, (path, rel_l2(got, want))


@pytest.mark.parametrize("tt", TYPES)
def test_every_launch_shape(gpu, oracle, tt):
    """Every tokens-per-pass variant, and lanes-per-row from 1 to one lane per
    chunk and beyond, including uneven splits of the chunks over the lanes."""
    rows, cols, tokens = 130, 2560 if tt != po.TT_Q6_K else 4096, 5
    w, x, wd, xd = setup(tt, rows, cols, tokens, gpu, seed=3)
    want = oracle.matvec(tt, w, x)
    xq = ops.quantize_act(tt, xd)
    units = cols // 64
    shapes = [(1, 1), (1, 2), (1, 4), (2, 1), (4, 1), (2, 2), (1, 8), (2, 4), (4, 4), (2, 8), (4, 8)]  # (rows/lane, tokens/pass)
    for lpr in sorted({1, 2, 3, 4, 7, 13, 31, 40, 64, units - 1}):
        for nr, tpp in shapes:
            got = ops.gemv_tuned(tt, wd, xq, rows, cols, tokens, lpr, tpp, nr).cpu().numpy()
            assert rel_l2(got, want) < TOL, (lpr, nr, tpp, rel_l2(got, want))


@pytest.mark.parametrize("tt", TYPES)
def test_unaligned_pointers_take_generic_path(gpu, oracle, tt):
    rows, cols = 24, 512
    w, x, _, xd = setup(tt, rows, cols, 2, gpu, seed=8)
    want = oracle.matvec(tt, w, x)
    xq = ops.quantize_act(tt, xd)
    wbuf = torch.zeros(w.size + 2, dtype=torch.uint8, device=gpu)
    wbuf[2:] = to_dev(w.reshape(-1), gpu)
    xbuf = torch.zeros(xq.numel() + 2, dtype=torch.uint8, device=gpu)
    xbuf[2:] = xq.reshape(-1)
    got = ops.mul_mat(tt, wbuf[2:], xbuf[2:], rows, cols, 2).cpu().numpy()
    assert rel_l2(got, want) < TOL


def test_q6_k_odd_total_bytes_uses_generic(gpu, oracle):
    # 9 super-blocks per row x 3 rows: total bytes % 4 == 2 -> generic kernel
    tt, rows, cols = po.TT_Q6_K, 3, 2304
    w, x, wd, xd = setup(tt, rows, cols, 1, gpu, seed=6)
    want = oracle.matvec(tt, w, x)
    xq = ops.quantize_act(tt, xd)
    got = ops.mul_mat(tt, wd, xq, rows, cols, 1).cpu().numpy()
    assert rel_l2(got, want) < TOL
    from qwen35_amd import _lib
    rc = _lib.load().qhip_launch_gemv_tuned(wd.data_ptr(), xq.data_ptr(), torch.empty(3, device=gpu).data_ptr(),
                                           rows, cols, 1, tt, 4, 1, 1, None)
    assert rc == -1  # fast path declines
    # the parity export serves only the fast-path layout
    rc = _lib.load().qhip_launch_block_ints(wd.data_ptr(), xq.data_ptr(), torch.empty(64, device=gpu).data_ptr(),
                                           rows, cols, 1, tt, None)
    assert rc == 1


def test_zero_weights_and_zero_activation(gpu, oracle):
    tt, rows, cols = po.TT_Q4_K, 16, 512
    w, x, wd, _ = setup(tt, rows, cols, 1, gpu)
    xq = ops.quantize_act(tt, torch.zeros((1, cols), device=gpu))
    assert torch.count_nonzero(ops.mul_mat(tt, wd, xq, rows, cols, 1)) == 0



# ---- quantize + GEMV in one launch -----------------------------------------------------

FUSED = [(po.TT_Q8_0, 300, 1024), (po.TT_Q8_0, 6144, 1024), (po.TT_IQ4_NL, 200, 2560),
         (po.TT_Q4_K, 100, 2560), (po.TT_Q4_K, 19456, 2560), (po.TT_Q6_K, 50, 9728),
         (po.TT_Q6_K, 2560, 9728), (po.TT_Q6_K, 16, 2304), (po.TT_Q5_K, 100, 2560), (po.TT_Q3_K, 60, 2304),
         (po.TT_Q2_K, 70, 2560), (po.TT_IQ4_XS, 80, 2560), (po.TT_Q4_0, 200, 2560),
         (po.TT_Q4_1, 150, 2560), (po.TT_Q4_1, 4096, 1024), (po.TT_IQ3_XXS, 90, 2560),
         (po.TT_IQ3_XXS, 6144, 2560), (po.TT_IQ3_S, 90, 2560), (po.TT_IQ3_S, 16, 2304)]


@pytest.mark.parametrize("tt,rows,cols", FUSED, ids=[case_id(*c) for c in FUSED])
def test_fused_quantize_gemv(gpu, oracle, tt, rows, cols):
    w = synth.make_weight(tt, rows, cols, seed=11, tag=tt)
    x = synth.make_act(cols, 1, seed=11)
    want = oracle.matvec(tt, w, x)[0]
    wd = to_dev(w, gpu)
    xq = torch.empty(oracle.quantize_act(tt, x).shape[-1], dtype=torch.uint8, device=gpu)
    got = ops.quantize_mul_mat_vec(tt, wd, to_dev(x[0], gpu), rows, cols, xq_out=xq).cpu().numpy()
    assert np.array_equal(xq.cpu().numpy(), oracle.quantize_act(tt, x)[0])
    assert rel_l2(got, want) < TOL
    # same numbers as the two-launch path
    two = ops.mul_mat(tt, wd, ops.quantize_act(tt, to_dev(x, gpu)), rows, cols, 1).cpu().numpy()[0]
    assert rel_l2(got, two) < 1e-6


FUSED_SHAPES = [(20, 1, 1024), (16, 2, 1024), (40, 2, 512), (8, 1, 512), (64, 4, 256), (12, 2, 256), (0, 0, 0)]


@pytest.mark.parametrize("tt,rows,cols", [(po.TT_Q4_K, 1000, 2560), (po.TT_Q8_0, 333, 1024),
                                          (po.TT_Q6_K, 70, 2304), (po.TT_IQ4_NL, 129, 2560)])
def test_fused_explicit_shapes(gpu, oracle, tt, rows, cols):
    """Explicit lanes / rows per lane / workgroup sizes, rows not a multiple
    of any workgroup's rows."""
    w = synth.make_weight(tt, rows, cols, seed=19, tag=tt)
    x = synth.make_act(cols, 1, seed=19)
    want = oracle.matvec(tt, w, x)[0]
    xq_want = oracle.quantize_act(tt, x)[0]
    wd, xd = to_dev(w, gpu), to_dev(x[0], gpu)
    for lpr, nr, wgs in FUSED_SHAPES:
        xq = torch.zeros(xq_want.shape[-1], dtype=torch.uint8, device=gpu)
        got = ops.quantize_mul_mat_vec_tuned(tt, wd, xd, rows, cols, lpr, nr, wgs, xq_out=xq).cpu().numpy()
        assert np.array_equal(xq.cpu().numpy(), xq_want), (lpr, nr, wgs)
        assert rel_l2(got, want) < TOL, (lpr, nr, wgs, rel_l2(got, want))
    for bad in [(8, 4, 512), (8, 1, 384), (65, 1, 256), (8, 3, 256)]:
        with pytest.raises(qwen35_amd.QhipError):
            ops.quantize_mul_mat_vec_tuned(tt, wd, xd, rows, cols, *bad)


@pytest.mark.parametrize("tt", [po.TT_Q8_0, po.TT_Q4_K])
def test_fused_quantize_special_values(gpu, oracle, tt):
    rows, cols = 40, 2048
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(cols) * 10.0 ** rng.uniform(-20, 20, cols // 256).repeat(256)).astype(np.float32)
    x[5] = np.inf
    x[300] = -0.0
    x[700:740] = 0.0
    x[1024:1030] = np.float32([127, 63.5, -63.5, .5, -.5, 1.5])
    w = synth.make_weight(tt, rows, cols, seed=2, tag=tt)
    xq = torch.empty(oracle.quantize_act(tt, x[None]).shape[-1], dtype=torch.uint8, device=gpu)
    ops.quantize_mul_mat_vec(tt, to_dev(w, gpu), to_dev(x, gpu), rows, cols, xq_out=xq)
    assert np.array_equal(xq.cpu().numpy(), oracle.quantize_act(tt, x[None])[0])


def test_fused_declines(gpu):
    from qwen35_amd import _lib
    L = _lib.load()
    tt, rows, cols = po.TT_Q4_K, 8, 512
    w = torch.zeros(rows * 288, dtype=torch.uint8, device=gpu)
    xbuf = torch.zeros(cols + 4, device=gpu)
    out = torch.empty(rows, device=gpu)
    # activation not 16-byte aligned
    assert L.qhip_launch_quantize_mul_mat_vec(w.data_ptr(), xbuf[1:].data_ptr(), None, out.data_ptr(), rows,
                                              cols, tt, None) == qwen35_amd.DECLINE
    # too wide for the LDS image
    wide = 65536
    w2 = torch.zeros(2 * wide // 32 * 34, dtype=torch.uint8, device=gpu)
    x2 = torch.zeros(wide, device=gpu)
    assert L.qhip_launch_quantize_mul_mat_vec(w2.data_ptr(), x2.data_ptr(), None, out.data_ptr(), 2, wide,
                                              po.TT_Q8_0, None) == qwen35_amd.DECLINE
    # invalid type is an error, not a decline
    rc = L.qhip_launch_quantize_mul_mat_vec(w.data_ptr(), xbuf.data_ptr(), None, out.data_ptr(), rows, cols, 99,
                                            None)
    assert rc not in (0, qwen35_amd.DECLINE)


# ---- split-K quantize + GEMV ---------------------------------------------------------

SPLIT = [(po.TT_Q6_K, 2560, 9728), (po.TT_Q6_K, 37, 9728), (po.TT_Q4_K, 300, 5120), (po.TT_Q5_K, 100, 4352),
         (po.TT_Q3_K, 60, 2304), (po.TT_Q2_K, 70, 2560), (po.TT_IQ4_XS, 80, 2560), (po.TT_IQ3_XXS, 90, 2560),
         (po.TT_IQ3_S, 16, 2304), (po.TT_Q8_0, 300, 2048), (po.TT_IQ4_NL, 200, 1024), (po.TT_Q4_0, 50, 2560),
         (po.TT_Q4_1, 70, 1536), (po.TT_Q6_K, 40, 17408), (po.TT_Q6_K, 36, 12288), (po.TT_Q4_K, 44, 16384)]
# (slice values, lanes per row, rows per lane); 0 picks.  768 leaves a short
# last slice on most widths; 64 lanes on a 256-value slice idle most lanes;
# 4096 / 16 and 2048 / 16 are the Q6_K defaults from widths 16384 / 12288
# (one slice, or a short last one, on narrower rows).
SPLIT_SHAPES = [(0, 0, 0), (256, 4, 1), (512, 8, 2), (768, 32, 2), (1024, 16, 4), (256, 64, 1), (2048, 64, 4),
                (4096, 16, 1), (2048, 16, 1)]


@pytest.mark.parametrize("tt,rows,cols", SPLIT, ids=[case_id(*c) for c in SPLIT])
def test_split_quantize_gemv(gpu, oracle, tt, rows, cols):
    w = synth.make_weight(tt, rows, cols, seed=13, tag=tt)
    x = synth.make_act(cols, 1, seed=13)
    want = oracle.matvec(tt, w, x)[0]
    xq_want = oracle.quantize_act(tt, x)[0]
    wd, xd = to_dev(w, gpu), to_dev(x[0], gpu)
    work = ops.split_work(rows, cols, gpu)
    first = None
    for sl, lpr, nr in SPLIT_SHAPES:
        xq = torch.zeros(xq_want.shape[-1], dtype=torch.uint8, device=gpu)
        got = ops.quantize_mul_mat_vec_split(tt, wd, xd, rows, cols, work, sl, lpr, nr, xq_out=xq).cpu().numpy()
        assert np.array_equal(xq.cpu().numpy(), xq_want), (sl, lpr, nr)
        assert rel_l2(got, want) < TOL, (sl, lpr, nr, rel_l2(got, want))
        if (sl, lpr, nr) == (0, 0, 0):
            first = got
    # the counters are back at zero: a repeat gives the same bits, and so does
    # a smaller matrix (fewer row tiles) on the same workspace
    again = ops.quantize_mul_mat_vec_split(tt, wd, xd, rows, cols, work).cpu().numpy()
    assert np.array_equal(again, first)
    small = max(4, rows // 12 * 4)  # a multiple of 4 rows keeps the weight 4-byte aligned
    got = ops.quantize_mul_mat_vec_split(tt, wd[:small], xd, small,
                                         cols, work).cpu().numpy()
    assert rel_l2(got, want[:small]) < TOL
    assert np.array_equal(work[: 4 * 8192].cpu().numpy(), np.zeros(4 * 8192, np.uint8))


def test_split_declines(gpu):
    from qwen35_amd import _lib
    L = _lib.load()
    tt, rows, cols = po.TT_Q6_K, 8, 1024
    w = torch.zeros(rows * cols // 256 * 210, dtype=torch.uint8, device=gpu)
    xbuf = torch.zeros(cols + 4, device=gpu)
    out = torch.empty(rows, device=gpu)
    work = ops.split_work(rows, cols, gpu)
    n = work.numel()
    # activation not 16-byte aligned: decline
    assert L.qhip_launch_quantize_mul_mat_vec_split(w.data_ptr(), xbuf[1:].data_ptr(), None, out.data_ptr(), rows,
                                                    cols, tt, 0, 0, 0, work.data_ptr(), n, None) == qwen35_amd.DECLINE
    # width not a multiple of 256 (Q8_0 rows of 1056 values): decline
    w8 = torch.zeros(rows * 1056 // 32 * 34, dtype=torch.uint8, device=gpu)
    x8 = torch.zeros(1056, device=gpu)
    work8 = ops.split_work(rows, 1056, gpu)
    assert L.qhip_launch_quantize_mul_mat_vec_split(w8.data_ptr(), x8.data_ptr(), None, out.data_ptr(), rows, 1056,
                                                    po.TT_Q8_0, 0, 0, 0, work8.data_ptr(), work8.numel(),
                                                    None) == qwen35_amd.DECLINE
    # a workspace too small, a bad slice or shape: errors
    for args in [(0, 0, 0, n - 4), (300, 0, 0, n), (0, 12, 0, n), (0, 2, 0, n), (0, 0, 3, n)]:
        sl, lpr, nr, nb = args
        rc = L.qhip_launch_quantize_mul_mat_vec_split(w.data_ptr(), xbuf.data_ptr(), None, out.data_ptr(), rows, cols,
                                                      tt, sl, lpr, nr, work.data_ptr(), nb, None)
        assert rc not in (0, qwen35_amd.DECLINE), args


@pytest.mark.parametrize("tt", TYPES)
def test_multiwave_team_shapes(gpu, oracle, tt):
    """Teams of two / four whole waves (one token), rows not a multiple of the
    rows per team, and uneven splits of the units over the waves."""
    rows, cols = 37, (9728 if tt == po.TT_Q6_K else 5120)
    w, x, wd, xd = setup(tt, rows, cols, 1, gpu, seed=9)
    want = oracle.matvec(tt, w, x)
    xq = ops.quantize_act(tt, xd)
    for lpr in (128, 256):
        for nr in (1, 2, 4):
            got = ops.gemv_tuned(tt, wd, xq, rows, cols, 1, lpr, 1, nr).cpu().numpy()
            assert rel_l2(got, want) < TOL, (lpr, nr, rel_l2(got, want))
    # multi-wave teams serve one token only
    xq2 = ops.quantize_act(tt, to_dev(synth.make_act(cols, 2, seed=9), gpu))
    with pytest.raises(qwen35_amd.QhipError):
        ops.gemv_tuned(tt, wd, xq2, rows, cols, 2, 128, 1, 1)
