"""GPU parity: the int8-MFMA tile path (MMQ) against the CPU oracle, through
the C ABI.

Bar: float outputs within 1e-5 relative L2 of the oracle; with every scale
set to 1.0 the float result is the plain sum of the per-block integers, so
those cases pin the MMQ's block integers bit-exactly against the oracle's.
"""
import numpy as np
import pytest
import torch

import pyoracle as po
import qwen35_amd
from qwen35_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu

TOL = 1e-5
TILES = [(64, 64), (64, 128), (128, 64), (128, 128), (32, 128), (32, 64)]
F16_ONE = np.array([0x00, 0x3C], np.uint8)  # 1.0 as little-endian binary16


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


# rows / tokens not multiples of any tile, partial 256-value chunks for the
# 32-value formats (cols % 256 != 0), K-quants at several super-block counts
CASES = [
    (po.TT_Q8_0, 200, 320, 37),
    (po.TT_Q8_0, 130, 1024, 130),
    (po.TT_IQ4_NL, 96, 576, 70),
    (po.TT_IQ4_NL, 33, 2560, 20),
    (po.TT_Q4_K, 150, 512, 65),
    (po.TT_Q4_K, 64, 2560, 16),
    (po.TT_Q4_K, 200, 768, 130),   # >= 128 tokens: the weights-direct kernel by default
    (po.TT_Q4_K, 333, 512, 257),
    (po.TT_Q6_K, 100, 768, 40),
    (po.TT_Q6_K, 72, 2304, 129),
    (po.TT_Q5_K, 150, 512, 65),
    (po.TT_Q5_K, 64, 2560, 16),
    (po.TT_IQ4_XS, 130, 768, 70),
    (po.TT_IQ4_XS, 33, 2560, 20),
    (po.TT_Q4_0, 200, 320, 37),
    (po.TT_Q4_0, 64, 2560, 16),
    (po.TT_Q4_1, 96, 576, 70),
    (po.TT_Q4_1, 130, 1024, 130),
    (po.TT_IQ3_XXS, 150, 512, 65),
    (po.TT_IQ3_XXS, 64, 2560, 16),
    (po.TT_IQ3_S, 130, 768, 70),
    (po.TT_IQ3_S, 33, 2560, 20),
    (po.TT_IQ4_NL, 96, 1024, 100),   # small grids with 4+ chunks per tile
    (po.TT_Q4_0, 200, 1280, 75),     # an odd chunk count
    (po.TT_Q8_0, 70, 2048, 66),
    (po.TT_Q4_1, 64, 1024, 128),
    (po.TT_Q3_K, 150, 512, 65),
    (po.TT_Q3_K, 72, 2304, 129),
    (po.TT_Q2_K, 100, 768, 40),
    (po.TT_Q2_K, 64, 2560, 16),
]
IDS = [f"{po.NAMES[c[0]]}-{c[1]}x{c[2]}-t{c[3]}" for c in CASES]


@pytest.mark.parametrize("tt,rows,cols,tokens", CASES, ids=IDS)
def test_mmq_matches_oracle_every_tile(gpu, oracle, tt, rows, cols, tokens):
    w = synth.make_weight(tt, rows, cols, seed=tokens, tag=tt)
    x = synth.make_act(cols, tokens, seed=tokens)
    want = oracle.matvec(tt, w, x)
    wd = to_dev(w, gpu)
    xq = ops.quantize_act(tt, to_dev(x, gpu))
    for bt, br in TILES + [(0, 0)]:
        got = ops.mmq_tuned(tt, wd, xq, rows, cols, tokens, bt, br).cpu().numpy()
        assert rel_l2(got, want) < TOL, (bt, br, rel_l2(got, want))
    # the reference-named entry point and the automatic path agree
    out = torch.empty((tokens, rows), device=gpu)
    rc = _lib.load().qhip_launch_mul_mat_vec_tile(wd.data_ptr(), xq.data_ptr(), out.data_ptr(), rows, cols,
                                                 tokens, tt, None)
    assert rc == 0
    assert rel_l2(out.cpu().numpy(), want) < TOL
    assert rel_l2(ops.mul_mat(tt, wd, xq, rows, cols, tokens).cpu().numpy(), want) < TOL
    # with the split-K workspace (small grids cut K; deterministic slice order)
    work = ops.mul_mat_work(rows, cols, tokens, tt, gpu)
    a = ops.mul_mat_split(tt, wd, xq, rows, cols, tokens, work, 2).cpu().numpy()
    b = ops.mul_mat_split(tt, wd, xq, rows, cols, tokens, work, 2).cpu().numpy()
    assert rel_l2(a, want) < TOL
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def unit_scale_weight(tt, rows, cols, seed):
    w = synth.make_weight(tt, rows, cols, seed=seed, tag=tt).copy()
    be, bb = po.GEOM[tt]
    blk = w.reshape(rows, cols // be, bb)
    if tt in (po.TT_Q8_0, po.TT_IQ4_NL, po.TT_IQ4_XS, po.TT_Q4_0, po.TT_IQ3_XXS, po.TT_IQ3_S):
        blk[:, :, 0:2] = F16_ONE
    elif tt in (po.TT_Q4_K, po.TT_Q5_K, po.TT_Q4_1):  # d = 1 and dmin (Q4_1: m) = 1
        blk[:, :, 0:2] = F16_ONE
        blk[:, :, 2:4] = F16_ONE
    elif tt == po.TT_Q3_K:
        blk[:, :, 108:110] = F16_ONE
    elif tt == po.TT_Q2_K:  # d = 1 and dmin = 1
        blk[:, :, 80:82] = F16_ONE
        blk[:, :, 82:84] = F16_ONE
    else:
        blk[:, :, 208:210] = F16_ONE
    return w


def unit_scale_act(cols, tokens, seed):
    # integers in [-127, 127] with +-127 in every 32-value block: the Q8_0 and
    # Q8_K scales are both exactly 1.0 and the quantized values equal x
    rng = np.random.default_rng(seed)
    x = rng.integers(-127, 128, (tokens, cols)).astype(np.float32)
    x[:, ::32] = np.where(rng.random((tokens, cols // 32)) < 0.5, -127.0, 127.0)
    return x


@pytest.mark.parametrize("tt", [po.TT_Q8_0, po.TT_IQ4_NL, po.TT_Q4_K, po.TT_Q6_K, po.TT_Q5_K, po.TT_IQ4_XS,
                                po.TT_Q4_0, po.TT_Q4_1, po.TT_IQ3_XXS, po.TT_IQ3_S, po.TT_Q3_K, po.TT_Q2_K])
def test_mmq_block_integers_exact(gpu, oracle, tt):
    # IQ4_XS / IQ3: the super-block sums carry the scales (up to 31), so a
    # narrower width keeps every result below 2^24; IQ3_XXS's 1/4 leaves
    # quarter values, exact with one super-block
    cols = {po.TT_IQ4_XS: 512, po.TT_IQ3_S: 512, po.TT_IQ3_XXS: 256}.get(tt, 1024)
    rows, tokens = 96, 72
    w = unit_scale_weight(tt, rows, cols, seed=5)
    x = unit_scale_act(cols, tokens, seed=5)
    act = oracle.quantize_act(tt, x)
    ints = oracle.block_ints(tt, w, act, cols).astype(np.int64)  # [tokens][rows][nints]
    if tt in (po.TT_Q4_K, po.TT_Q5_K, po.TT_Q2_K):
        want = ints[:, :, 0::2].sum(-1) - ints[:, :, 1::2].sum(-1)  # isum - summs
    elif tt == po.TT_Q4_1:
        want = ints[:, :, 0::2].sum(-1) + ints[:, :, 1::2].sum(-1)  # sumi + sumy
    elif tt == po.TT_IQ4_XS:
        # per-block integers times the block's ls - 32 (d = 1, dy = 1)
        blk = w.reshape(rows, cols // 256, 136)
        sh = blk[:, :, 2].astype(np.int64) | (blk[:, :, 3].astype(np.int64) << 8)
        ls = np.stack([((blk[:, :, 4 + ib // 2] >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4)
                       for ib in range(8)], axis=-1).reshape(rows, -1) - 32
        want = (ints * ls[None, :, :]).sum(-1)
    elif tt in (po.TT_IQ3_XXS, po.TT_IQ3_S):
        # per-block integers times 2 ls + 1 (d = 1, dy = 1); IQ3_XXS times 1/4
        blk = w.reshape(rows, cols // 256, -1)
        if tt == po.TT_IQ3_XXS:
            ls = np.stack([blk[:, :, 66 + 4 * ib + 3] >> 4 for ib in range(8)], axis=-1)
        else:
            ls = np.stack([(blk[:, :, 106 + ib // 2] >> (4 * (ib % 2))) & 15 for ib in range(8)], axis=-1)
        want = (ints * (2 * ls.reshape(rows, -1).astype(np.int64) + 1)[None, :, :]).sum(-1)
    else:
        want = ints.sum(-1)
    assert np.abs(want).max() < 2 ** 24  # every partial float sum is exact
    xq = ops.quantize_act(tt, to_dev(x, gpu))
    assert np.array_equal(xq.cpu().numpy(), act)
    wd = to_dev(w, gpu)
    for bt, br in TILES:
        got = ops.mmq_tuned(tt, wd, xq, rows, cols, tokens, bt, br).cpu().numpy()
        if tt == po.TT_IQ3_XXS:
            got = got * np.float32(4.0)  # exact: the 1/4 is a power of two
        assert np.array_equal(got.astype(np.int64), want), (bt, br)
        assert np.array_equal(got, want.astype(np.float32))


@pytest.mark.parametrize("tt", [po.TT_Q8_0, po.TT_Q6_K])
def test_mmq_declines_unaligned(gpu, tt):
    rows, cols, tokens = 16, 512, 20
    w = synth.make_weight(tt, rows, cols, seed=1, tag=tt)
    x = synth.make_act(cols, tokens, seed=1)
    xq = ops.quantize_act(tt, to_dev(x, gpu))
    wbuf = torch.zeros(w.size + 2, dtype=torch.uint8, device=gpu)
    wbuf[2:] = to_dev(w.reshape(-1), gpu)
    out = torch.empty((tokens, rows), device=gpu)
    L = _lib.load()
    rc = L.qhip_launch_mmq_tuned(wbuf[2:].data_ptr(), xq.data_ptr(), out.data_ptr(), rows, cols, tokens, tt,
                                 64, 64, None)
    assert rc == qwen35_amd.DECLINE
    rc = L.qhip_launch_mul_mat_vec_tile(wbuf[2:].data_ptr(), xq.data_ptr(), out.data_ptr(), rows, cols,
                                        tokens, tt, None)
    assert rc == qwen35_amd.DECLINE
    # the automatic path still serves it (generic kernel)
    got = ops.mul_mat(tt, wbuf[2:], xq, rows, cols, tokens).cpu().numpy()
    assert rel_l2(got, po.Oracle().matvec(tt, w, x)) < TOL


def test_mmq_rejects_bad_tiles(gpu):
    tt, rows, cols, tokens = po.TT_Q4_K, 16, 256, 8
    w = torch.zeros(rows * 144, dtype=torch.uint8, device=gpu)
    xq = torch.zeros(tokens * 292, dtype=torch.uint8, device=gpu)
    out = torch.empty((tokens, rows), device=gpu)
    L = _lib.load()
    for bt, br in [(32, 32), (64, 256), (-1, 64), (16, 64)]:
        rc = L.qhip_launch_mmq_tuned(w.data_ptr(), xq.data_ptr(), out.data_ptr(), rows, cols, tokens, tt, bt,
                                     br, None)
        assert rc not in (0, qwen35_amd.DECLINE), (bt, br)


def test_mmq_zero_tokens_and_rows_are_noops(gpu):
    tt = po.TT_Q8_0
    w = torch.zeros(34 * 2, dtype=torch.uint8, device=gpu)
    xq = torch.zeros(34 * 2, dtype=torch.uint8, device=gpu)
    out = torch.full((1,), 7.0, device=gpu)
    L = _lib.load()
    assert L.qhip_launch_mmq_tuned(w.data_ptr(), xq.data_ptr(), out.data_ptr(), 1, 64, 0, tt, 0, 0, None) == 0
    assert L.qhip_launch_mmq_tuned(w.data_ptr(), xq.data_ptr(), out.data_ptr(), 0, 64, 1, tt, 0, 0, None) == 0
    assert out.item() == 7.0


def test_cfg4_ragged_batch_through_mmq(gpu, oracle):
    """BASELINE config 4 shape: eight sequences, lengths uniform on [16,256],
    packed with the offset table and multiplied in one launch."""
    tt, rows, cols = po.TT_Q8_0, 3584, 1024
    lens = [int(v) for v in synth.ragged_lengths(8, 16, 256, seed=0)]
    w = synth.make_weight(tt, rows, cols, seed=0, tag=tt)
    seqs = [synth.make_act(cols, n, seed=300 + i) for i, n in enumerate(lens)]
    dseqs = [to_dev(s, gpu) for s in seqs]
    xq, off_d, total = ops.quantize_ragged(tt, dseqs, cols)
    assert total == sum(lens)
    packed = np.concatenate(seqs)
    wd = to_dev(w, gpu)
    out = ops.mul_mat_ragged(tt, wd, xq, off_d, len(lens), total, rows, cols).cpu().numpy()
    # sampled rows of every token against the oracle (the full product is 1.1G MACs on the CPU)
    idx = np.unique(np.concatenate([[0, rows - 1], np.random.default_rng(4).integers(0, rows, 200)]))
    want = oracle.matvec(tt, np.ascontiguousarray(w[idx]), packed)
    assert rel_l2(out[:, idx], want) < TOL
    assert np.all(np.isfinite(out))


# ---- MMQ from the prepared weight image (Q4_K, Q6_K) ----------------------------------

def _q4k_p(w, cols):
    """p = sc * q for every value of Q4_K rows (kernels256.c:105-125, :179-186)."""
    blk = w.reshape(w.shape[0], cols // 256, 144).astype(np.int64)
    s12 = blk[:, :, 4:16]
    sc = np.empty(blk.shape[:2] + (8,), np.int64)
    for j in range(8):
        sc[:, :, j] = (s12[:, :, j] & 63) if j < 4 else ((s12[:, :, j + 4] & 15) | ((s12[:, :, j - 4] >> 6) << 4))
    qs = blk[:, :, 16:144].reshape(blk.shape[0], blk.shape[1], 4, 32)
    q = np.stack([qs & 15, qs >> 4], axis=3).reshape(blk.shape[0], blk.shape[1], 8, 32)  # sub-block 2c, 2c+1
    return (sc[:, :, :, None] * q).reshape(blk.shape[0], blk.shape[1], 256)


def _q6k_p(w, cols):
    """p = sc * (q6 - 32) for every value of Q6_K rows (kernels256.c:200-212, :720-738)."""
    blk = w.reshape(w.shape[0], cols // 256, 210).astype(np.int64)
    e = np.arange(256)
    h, q, l = e // 128, (e % 128) // 32, e % 32
    lo = blk[:, :, 64 * h + 32 * (q & 1) + l]
    lo = np.where(q >= 2, lo >> 4, lo & 15)
    hb = (blk[:, :, 128 + 32 * h + l] >> (2 * q)) & 3
    sc = blk[:, :, 192 + e // 16].astype(np.int8).astype(np.int64)
    return sc * ((lo | (hb << 4)) - 32)


@pytest.mark.parametrize("tt", [po.TT_Q4_K, po.TT_Q6_K])
def test_mmq_image_planes(gpu, tt):
    rows, cols = 9 if tt == po.TT_Q4_K else 45, 1024
    w = synth.make_weight(tt, rows, cols, seed=12, tag=tt)
    img = ops.mmq_image(tt, to_dev(w, gpu), rows, cols).cpu().numpy()
    nsb = cols // 256
    p = _q4k_p(w, cols) if tt == po.TT_Q4_K else _q6k_p(w, cols)
    if tt == po.TT_Q4_K:
        planes = img[:rows * nsb * 512].reshape(rows, nsb, 512)
        S = 7
        hi = planes[:, :, :256].view(np.int8).astype(np.int64)
        lo = planes[:, :, 256:].astype(np.int64)
    else:
        # per 32-row group and super-block: hi fragments [s][lane][16], lo
        # fragments, then the 32 rows' f32 d; lane L holds row L % 32, values
        # 32 s + 16 (L // 32) .. +15
        S = 6
        ngrp = -(-rows // 32)
        g = img.reshape(ngrp, nsb, 16512)
        fr = g[:, :, :16384].reshape(ngrp, nsb, 2, 8, 2, 32, 16)  # plane, s, L // 32, L % 32, byte
        fr = fr.transpose(2, 0, 5, 1, 3, 4, 6).reshape(2, ngrp * 32, nsb, 256)[:, :rows]
        hi = fr[0].view(np.int8).astype(np.int64)
        lo = fr[1].astype(np.int64)
        d = g[:, :, 16384:].copy().view(np.float32).transpose(0, 2, 1).reshape(ngrp * 32, nsb)
        blk = w.reshape(rows, nsb, 210)
        assert np.array_equal(d[:rows], blk[:, :, 208:210].copy().view(np.float16)[..., 0].astype(np.float32))
        assert not d[rows:].any()
    assert np.array_equal(hi * (1 << S) + lo, p)
    assert lo.min() >= 0 and lo.max() < (1 << S) and hi.min() >= -128 and hi.max() <= 127
    if tt == po.TT_Q4_K:
        hdr = img[rows * nsb * 512:].reshape(rows, nsb, 48)
        d = hdr[:, :, 32:36].copy().view(np.float32)[..., 0]
        dmin = hdr[:, :, 36:40].copy().view(np.float32)[..., 0]
        blk = w.reshape(rows, nsb, 144)
        assert np.array_equal(d, blk[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float32))
        assert np.array_equal(dmin, blk[:, :, 2:4].copy().view(np.float16)[..., 0].astype(np.float32))
        mins = hdr[:, :, 0:32].copy().view(np.float16).astype(np.int64)  # [rows, nsb, 16]
        s12 = blk[:, :, 4:16].astype(np.int64)
        for j in range(16):
            k = j // 2
            m = (s12[:, :, k + 4] & 63) if k < 4 else ((s12[:, :, k + 4] >> 4) | ((s12[:, :, k] >> 6) << 4))
            assert np.array_equal(mins[:, :, j], m)
    else:
        # the padding rows of the last group are zeros
        pad = img.reshape(-1, nsb, 16512)[-1, :, :16384].reshape(nsb, 2, 8, 2, 32, 16)[:, :, :, :, rows % 32:]
        assert not pad.any()


# Q6_K: 64-token tiles (<= 192 tokens) and 128-token tiles, rows and tokens
# off every tile size, grids whose tiles are cut over K
IMG_CASES = [(po.TT_Q4_K, 150, 512, 65), (po.TT_Q4_K, 64, 2560, 16), (po.TT_Q6_K, 100, 768, 40),
             (po.TT_Q6_K, 72, 2304, 129), (po.TT_Q6_K, 200, 2304, 300), (po.TT_Q6_K, 333, 4608, 70),
             (po.TT_Q6_K, 40, 1024, 193), (po.TT_Q6_K, 129, 2560, 1)]


@pytest.mark.parametrize("tt,rows,cols,tokens", IMG_CASES,
                         ids=[f"{po.NAMES[c[0]]}-{c[1]}x{c[2]}-t{c[3]}" for c in IMG_CASES])
def test_mmq_image_matches_oracle(gpu, oracle, tt, rows, cols, tokens):
    w = synth.make_weight(tt, rows, cols, seed=tokens + 1, tag=tt)
    x = synth.make_act(cols, tokens, seed=tokens + 1)
    want = oracle.matvec(tt, w, x)
    img = ops.mmq_image(tt, to_dev(w, gpu), rows, cols)
    xq = ops.quantize_act(tt, to_dev(x, gpu))
    tiles = [(64, 64), (64, 128), (128, 64), (0, 0)] if tt == po.TT_Q4_K else [(0, 0)]
    for bt, br in tiles:
        got = ops.mul_mat_image(tt, img, xq, rows, cols, tokens, bt, br).cpu().numpy()
        assert rel_l2(got, want) < TOL, (bt, br, rel_l2(got, want))
    work = ops.mul_mat_work(rows, cols, tokens, tt, gpu)
    got = ops.mul_mat_image(tt, img, xq, rows, cols, tokens, work=work).cpu().numpy()
    assert rel_l2(got, want) < TOL
    if tt == po.TT_Q6_K:
        # one shape only: an explicit tile is refused before any launch
        L = _lib.load()
        out = torch.empty((tokens, rows), device=gpu)
        assert L.qhip_launch_mul_mat_image(img.data_ptr(), xq.data_ptr(), out.data_ptr(), rows, cols, tokens, tt,
                                           64, 64, None, 0, None) == 1  # hipErrorInvalidValue


@pytest.mark.parametrize("tt", [po.TT_Q4_K, po.TT_Q6_K])
def test_mmq_image_block_integers_exact(gpu, oracle, tt):
    rows, cols, tokens = 96, 1024, 72
    w = unit_scale_weight(tt, rows, cols, seed=7)
    x = unit_scale_act(cols, tokens, seed=7)
    act = oracle.quantize_act(tt, x)
    ints = oracle.block_ints(tt, w, act, cols).astype(np.int64)
    want = ints[:, :, 0::2].sum(-1) - ints[:, :, 1::2].sum(-1) if tt == po.TT_Q4_K else ints.sum(-1)
    assert np.abs(want).max() < 2 ** 24
    img = ops.mmq_image(tt, to_dev(w, gpu), rows, cols)
    xq = ops.quantize_act(tt, to_dev(x, gpu))
    got = ops.mul_mat_image(tt, img, xq, rows, cols, tokens).cpu().numpy()
    assert np.array_equal(got, want.astype(np.float32))


def test_mmq_image_rejects_other_types(gpu):
    L = _lib.load()
    assert L.qhip_mmq_image_bytes(po.TT_Q8_0, 4, 1024) == -1
    assert L.qhip_mmq_image_bytes(po.TT_Q4_K, 4, 1000) == -1
    assert L.qhip_mmq_image_bytes(po.TT_Q4_K, 4, 1024) == 4 * 4 * 560
    assert L.qhip_mmq_image_bytes(po.TT_Q6_K, 4, 1024) == 1 * 4 * 16512
    assert L.qhip_mmq_image_bytes(po.TT_Q6_K, 33, 1024) == 2 * 4 * 16512
    w = torch.zeros(4 * 34 * 32, dtype=torch.uint8, device=gpu)
    img = torch.empty(4096, dtype=torch.uint8, device=gpu)
    assert L.qhip_launch_mmq_prepare(po.TT_Q8_0, w.data_ptr(), 4, 1024, img.data_ptr(), None) != 0


@pytest.mark.parametrize("tt", [po.TT_Q4_K, po.TT_Q6_K])
def test_backend_prefill_batch(gpu, oracle, tt):
    """matvecBatchK above the crossover: the MMQ image for Q6_K (the plane
    image, from 64 tokens), the tile MMQ for Q4_K; the second call reuses the
    cached image."""
    rows, cols, k = 130, 2560 if tt == po.TT_Q4_K else 2304, 80 if tt == po.TT_Q4_K else 130
    w = synth.make_weight(tt, rows, cols, seed=31, tag=tt)
    x = synth.make_act(cols, k, seed=31)
    be = ops.Backend(0)
    try:
        lin = be.load_linear(tt, rows, cols, w)
        out = torch.empty((k, rows), device=gpu)
        for rep in range(2):
            out.zero_()
            be.matvec_batch_k(out, lin, to_dev(x, gpu), k)
            be.sync()
            assert rel_l2(out.cpu().numpy(), oracle.matvec(tt, w, x)) < TOL, rep
        be.lib.qhip_backend_free_linear(be._h, ctypes_byref(lin))
    finally:
        be.close()


def ctypes_byref(x):
    import ctypes
    return ctypes.byref(x)


@pytest.mark.parametrize("tt", [po.TT_Q3_K, po.TT_Q2_K])
def test_q3_k_q2_k_mmq_entry_points(gpu, oracle, tt):
    """Q3_K / Q2_K: the reference-named tile entry point and the automatic
    path take the MMQ; there is no weight image for them."""
    rows, cols, tokens = 72, 1024, 70
    w = synth.make_weight(tt, rows, cols, seed=12, tag=tt)
    x = synth.make_act(cols, tokens, seed=12)
    wd = to_dev(w, gpu)
    xq = ops.quantize_act(tt, to_dev(x, gpu))
    out = torch.empty((tokens, rows), device=gpu)
    L = _lib.load()
    want = oracle.matvec(tt, w, x)
    assert L.qhip_launch_mul_mat_vec_tile(wd.data_ptr(), xq.data_ptr(), out.data_ptr(), rows, cols, tokens, tt,
                                          None) == 0
    assert rel_l2(out.cpu().numpy(), want) < TOL
    assert L.qhip_mmq_image_bytes(tt, rows, cols) == -1
    got = ops.mul_mat(tt, wd, xq, rows, cols, tokens).cpu().numpy()
    assert rel_l2(got, oracle.matvec(tt, w, x)) < TOL
