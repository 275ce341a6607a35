"""GPU: the default MMQ launches that pick their own kernel and K split --
the weights-direct Q4_K kernel (its few-token variant up to 24 tokens,
32-token tiles up to 32 and from 65 to 96, 64-token tiles otherwise; K split
over workgroups on small grids and to fill whole rounds with several token
tiles), the
few-token weights-direct Q6_K kernel (up to 24 tokens) and the Q6_K image --
against the oracle at token counts either side of every switch with
row counts that are no multiple of a tile; exact block integers at unit
scales on the default path; and the same bits on every rerun (the slices of
a split are added in a fixed order)."""
import numpy as np
import pytest
import torch

import pyoracle as po
from qwen35_amd import ops, synth
from test_gpu_mmq import rel_l2, to_dev, unit_scale_act, unit_scale_weight

pytestmark = pytest.mark.gpu
TOL = 1e-5
PATH_MMQ = 2

Q4K_T = [1, 2, 3, 5, 8, 9, 16, 17, 24, 25, 31, 32, 33, 63, 64, 65, 96, 97, 128, 130]


@pytest.fixture(scope="module")
def q4k(gpu):
    rows, cols = 333, 5120
    w = synth.make_weight(po.TT_Q4_K, rows, cols, seed=31, tag=po.TT_Q4_K)
    return rows, cols, w, to_dev(w, gpu)


@pytest.mark.parametrize("tokens", Q4K_T)
def test_q4k_default_mmq_every_token_count(gpu, oracle, q4k, tokens):
    rows, cols, w, wd = q4k
    x = synth.make_act(cols, tokens, seed=32, tag=tokens)
    xq = ops.quantize_act(po.TT_Q4_K, to_dev(x, gpu))
    work = ops.mul_mat_work(rows, cols, tokens, po.TT_Q4_K, gpu)
    got = ops.mul_mat_split(po.TT_Q4_K, wd, xq, rows, cols, tokens, work, PATH_MMQ)
    assert rel_l2(got.cpu().numpy(), oracle.matvec(po.TT_Q4_K, w, x)) < TOL
    again = ops.mul_mat_split(po.TT_Q4_K, wd, xq, rows, cols, tokens, work, PATH_MMQ)
    assert torch.equal(got, again)
    # without a workspace the launch is not split: same integers, same tolerance
    plain = ops.mul_mat(po.TT_Q4_K, wd, xq, rows, cols, tokens, PATH_MMQ)
    assert rel_l2(plain.cpu().numpy(), got.cpu().numpy()) < 1e-6


@pytest.mark.parametrize("tokens", [3, 8, 20, 30, 40, 72])
def test_q4k_default_mmq_integers_exact(gpu, oracle, tokens):
    """d = dmin = 1 and activations of Q8_K scale 1: every output is the exact
    isum - summs of its row, on each of the default path's kernels."""
    rows, cols = 96, 1024
    w = unit_scale_weight(po.TT_Q4_K, rows, cols, seed=33)
    x = unit_scale_act(cols, tokens, seed=33)
    act = oracle.quantize_act(po.TT_Q4_K, x)
    ints = oracle.block_ints(po.TT_Q4_K, w, act, cols).astype(np.int64)
    want = ints[:, :, 0::2].sum(-1) - ints[:, :, 1::2].sum(-1)
    assert np.abs(want).max() < 2 ** 24
    xq = ops.quantize_act(po.TT_Q4_K, to_dev(x, gpu))
    work = ops.mul_mat_work(rows, cols, tokens, po.TT_Q4_K, gpu)
    got = ops.mul_mat_split(po.TT_Q4_K, to_dev(w, gpu), xq, rows, cols, tokens, work, PATH_MMQ).cpu().numpy()
    assert np.array_equal(got, want.astype(np.float32))


@pytest.mark.parametrize("tt,rows,cols,tokens", [(po.TT_Q4_K, 700, 2560, 96), (po.TT_Q4_K, 700, 2560, 200),
                                                 (po.TT_Q4_K, 300, 2560, 257), (po.TT_Q6_K, 200, 2304, 96),
                                                 (po.TT_Q6_K, 200, 2304, 129), (po.TT_Q6_K, 130, 2304, 300)])
def test_round_filling_split(gpu, oracle, tt, rows, cols, tokens):
    """Several token tiles on a small grid: the launch splits K to fill whole
    rounds of resident workgroups (the Q6_K case through its MMQ image)."""
    w = synth.make_weight(tt, rows, cols, seed=34, tag=tt)
    x = synth.make_act(cols, tokens, seed=34, tag=tokens)
    xq = ops.quantize_act(tt, to_dev(x, gpu))
    work = ops.mul_mat_work(rows, cols, tokens, tt, gpu)
    assert work is not None  # these grids are small enough to split
    wd = to_dev(w, gpu)
    if tt == po.TT_Q6_K:
        img = ops.mmq_image(tt, wd, rows, cols)
        run = lambda: ops.mul_mat_image(tt, img, xq, rows, cols, tokens, work=work)  # noqa: E731
    else:
        run = lambda: ops.mul_mat_split(tt, wd, xq, rows, cols, tokens, work, PATH_MMQ)  # noqa: E731
    got = run()
    assert rel_l2(got.cpu().numpy(), oracle.matvec(tt, w, x)) < TOL
    assert torch.equal(got, run())


Q6K_T = [1, 2, 3, 7, 8, 9, 15, 16, 17, 23, 24, 25, 32]


@pytest.fixture(scope="module")
def q6k(gpu):
    rows, cols = 333, 4608
    w = synth.make_weight(po.TT_Q6_K, rows, cols, seed=35, tag=po.TT_Q6_K)
    return rows, cols, w, to_dev(w, gpu)


@pytest.mark.parametrize("tokens", Q6K_T)
def test_q6k_default_mmq_few_tokens(gpu, oracle, q6k, tokens):
    """The few-token weights-direct Q6_K kernel up to 24 tokens (K split over
    the small grid), the 32-token tile kernel beyond."""
    rows, cols, w, wd = q6k
    x = synth.make_act(cols, tokens, seed=36, tag=tokens)
    xq = ops.quantize_act(po.TT_Q6_K, to_dev(x, gpu))
    work = ops.mul_mat_work(rows, cols, tokens, po.TT_Q6_K, gpu)
    got = ops.mul_mat_split(po.TT_Q6_K, wd, xq, rows, cols, tokens, work, PATH_MMQ)
    assert rel_l2(got.cpu().numpy(), oracle.matvec(po.TT_Q6_K, w, x)) < TOL
    assert torch.equal(got, ops.mul_mat_split(po.TT_Q6_K, wd, xq, rows, cols, tokens, work, PATH_MMQ))
    plain = ops.mul_mat(po.TT_Q6_K, wd, xq, rows, cols, tokens, PATH_MMQ)
    assert rel_l2(plain.cpu().numpy(), got.cpu().numpy()) < 1e-6


@pytest.mark.parametrize("tokens", [1, 5, 8, 13, 24])
def test_q6k_default_mmq_integers_exact(gpu, oracle, tokens):
    """d = 1 and activations of Q8_K scale 1: every output is the exact sum of
    its row's block integers (the -32 offset through the scaled bsums)."""
    rows, cols = 96, 1024
    w = unit_scale_weight(po.TT_Q6_K, rows, cols, seed=37)
    x = unit_scale_act(cols, tokens, seed=37)
    act = oracle.quantize_act(po.TT_Q6_K, x)
    want = oracle.block_ints(po.TT_Q6_K, w, act, cols).astype(np.int64).sum(-1)
    assert np.abs(want).max() < 2 ** 24
    xq = ops.quantize_act(po.TT_Q6_K, to_dev(x, gpu))
    work = ops.mul_mat_work(rows, cols, tokens, po.TT_Q6_K, gpu)
    wd = to_dev(w, gpu)
    for wk in (work, None):
        got = ops.mul_mat_split(po.TT_Q6_K, wd, xq, rows, cols, tokens, wk, PATH_MMQ).cpu().numpy()
        assert np.array_equal(got, want.astype(np.float32))


def test_q6k_few_token_extreme_values(gpu, oracle):
    """Every 6-bit value 0 and 63, scales -128 and 127, activations +-127:
    the largest products the kernel's integer and f16 sums meet."""
    rows, cols, tokens = 64, 2048, 8
    w = unit_scale_weight(po.TT_Q6_K, rows, cols, seed=38).reshape(rows, -1, 210)
    rng = np.random.default_rng(38)
    w[:, :, 0:192] = np.where(rng.random((rows, w.shape[1], 192)) < 0.5, 0x00, 0xFF).astype(np.uint8)
    w[:, :, 192:208] = np.where(rng.random((rows, w.shape[1], 16)) < 0.5, 0x80, 0x7F).astype(np.uint8)
    w = w.reshape(rows, -1)
    x = np.where(rng.random((tokens, cols)) < 0.5, -127.0, 127.0).astype(np.float32)
    act = oracle.quantize_act(po.TT_Q6_K, x)
    xq = ops.quantize_act(po.TT_Q6_K, to_dev(x, gpu))
    work = ops.mul_mat_work(rows, cols, tokens, po.TT_Q6_K, gpu)
    got = ops.mul_mat_split(po.TT_Q6_K, to_dev(w, gpu), xq, rows, cols, tokens, work, PATH_MMQ).cpu().numpy()
    ints = oracle.block_ints(po.TT_Q6_K, w, act, cols).astype(np.int64)
    assert 2 ** 24 < np.abs(ints).max() < 2 ** 31  # past f32's integers, inside int32
    assert rel_l2(got, oracle.matvec(po.TT_Q6_K, w, x)) < TOL
    # each super-block's integer is exact and rounded once to f32, as the
    # reference's (float)isum; their f32 sum is within rounding
    assert rel_l2(got, ints.astype(np.float32).astype(np.float64).sum(-1)) < 1e-6
