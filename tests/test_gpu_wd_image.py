"""GPU: the Q6_K and Q4_K fragment images -- their layouts restated on the
host from the GGUF bytes, the weights-direct MMQ read from them against the
oracle at token counts either side of each kernel variant and row counts off
the 32-row groups, the same bits as the GGUF-row kernels, exact block
integers at unit scales, extreme 6-bit values and scales, bit-equal reruns,
and the Exec mirror reading the Q6_K image."""
import numpy as np
import pytest
import torch

import pyoracle as po
from qwen35_amd import _lib, ops, synth
from test_gpu_mmq import rel_l2, to_dev, unit_scale_act, unit_scale_weight

pytestmark = pytest.mark.gpu
TOL = 1e-5
PATH_MMQ = 2
TQ6 = po.TT_Q6_K
TQ4 = po.TT_Q4_K


def wd_image_of(w, rows, cols):
    """The documented fragment-image layout, from the GGUF bytes."""
    nsb = cols // 256
    ngrp = (rows + 31) // 32
    pad = np.zeros((ngrp * 32, nsb, 210), np.uint8)
    pad[:rows] = w.reshape(rows, nsb, 210)
    img = np.zeros((ngrp, nsb, 6720), np.uint8)
    for k in range(2):
        pieces = []
        for j in range(4):
            h, m = j >> 1, j & 1
            for off in (64 * h + 16 * m + 8 * k, 64 * h + 32 + 16 * m + 8 * k, 128 + 32 * h + 16 * m + 8 * k):
                pieces.append(pad[:, :, off:off + 8])
        lane = np.concatenate(pieces, axis=-1).reshape(ngrp, 32, nsb, 96)
        for c in range(6):
            img[:, :, 1024 * c + 512 * k:1024 * c + 512 * (k + 1)] = \
                lane[:, :, :, 16 * c:16 * c + 16].transpose(0, 2, 1, 3).reshape(ngrp, nsb, 512)
    img[:, :, 6144:6656] = pad[:, :, 192:208].reshape(ngrp, 32, nsb, 16).transpose(0, 2, 1, 3).reshape(ngrp, nsb, 512)
    img[:, :, 6656:6720] = pad[:, :, 208:210].reshape(ngrp, 32, nsb, 2).transpose(0, 2, 1, 3).reshape(ngrp, nsb, 64)
    return img.reshape(-1)


@pytest.mark.parametrize("rows,cols", [(1, 256), (31, 512), (32, 2304), (33, 256), (70, 1024)])
def test_wd_image_layout(gpu, rows, cols):
    w = synth.make_weight(TQ6, rows, cols, seed=40, tag=rows)
    n = ops.load().qhip_wd_image_bytes(TQ6, rows, cols)
    assert n == (rows + 31) // 32 * (cols // 256) * 6720
    img = ops.wd_image(TQ6, to_dev(w, gpu), rows, cols).cpu().numpy()
    assert np.array_equal(img[:n], wd_image_of(w, rows, cols))


@pytest.fixture(scope="module")
def q6(gpu):
    rows, cols = 333, 4608
    w = synth.make_weight(TQ6, rows, cols, seed=41, tag=TQ6)
    wd = to_dev(w, gpu)
    return rows, cols, w, wd, ops.wd_image(TQ6, wd, rows, cols)


@pytest.mark.parametrize("tokens", [1, 2, 3, 7, 8, 9, 16, 17, 24, 25, 31, 32, 33, 40, 63, 64])
def test_wd_image_mmq_vs_oracle(gpu, oracle, q6, tokens):
    rows, cols, w, wd, img = q6
    x = synth.make_act(cols, tokens, seed=42, tag=tokens)
    xq = ops.quantize_act(TQ6, to_dev(x, gpu))
    work = ops.mul_mat_work(rows, cols, tokens, TQ6, gpu)
    got = ops.mul_mat_wd_image(TQ6, img, xq, rows, cols, tokens, work)
    assert rel_l2(got.cpu().numpy(), oracle.matvec(TQ6, w, x)) < TOL
    assert torch.equal(got, ops.mul_mat_wd_image(TQ6, img, xq, rows, cols, tokens, work))
    # without a workspace: not split, the same integers
    plain = ops.mul_mat_wd_image(TQ6, img, xq, rows, cols, tokens)
    assert rel_l2(plain.cpu().numpy(), got.cpu().numpy()) < 1e-6
    if tokens <= 24:
        # the GGUF-row few-token kernel: the same block integers; from 17
        # tokens the same slices in the same order (up to 16 the image's
        # launch adds its K pieces inside the workgroup)
        raw = ops.mul_mat_split(TQ6, wd, xq, rows, cols, tokens, work, PATH_MMQ)
        if tokens > 16:
            assert torch.equal(got, raw)
        else:
            assert rel_l2(got.cpu().numpy(), raw.cpu().numpy()) < 1e-6


@pytest.mark.parametrize("tokens", [1, 6, 8, 19, 32, 45, 64])
def test_wd_image_integers_exact(gpu, oracle, tokens):
    rows, cols = 96, 1024
    w = unit_scale_weight(TQ6, rows, cols, seed=43)
    x = unit_scale_act(cols, tokens, seed=43)
    act = oracle.quantize_act(TQ6, x)
    want = oracle.block_ints(TQ6, w, act, cols).astype(np.int64).sum(-1)
    assert np.abs(want).max() < 2 ** 24
    img = ops.wd_image(TQ6, to_dev(w, gpu), rows, cols)
    xq = ops.quantize_act(TQ6, to_dev(x, gpu))
    work = ops.mul_mat_work(rows, cols, tokens, TQ6, gpu)
    for wk in (work, None):
        got = ops.mul_mat_wd_image(TQ6, img, xq, rows, cols, tokens, wk).cpu().numpy()
        assert np.array_equal(got, want.astype(np.float32))


def test_wd_image_extreme_values(gpu, oracle):
    rows, cols, tokens = 40, 2048, 12
    w = unit_scale_weight(TQ6, rows, cols, seed=44).reshape(rows, -1, 210)
    rng = np.random.default_rng(44)
    w[:, :, 0:192] = np.where(rng.random((rows, w.shape[1], 192)) < 0.5, 0x00, 0xFF).astype(np.uint8)
    w[:, :, 192:208] = np.where(rng.random((rows, w.shape[1], 16)) < 0.5, 0x80, 0x7F).astype(np.uint8)
    w = w.reshape(rows, -1)
    x = np.where(rng.random((tokens, cols)) < 0.5, -127.0, 127.0).astype(np.float32)
    img = ops.wd_image(TQ6, to_dev(w, gpu), rows, cols)
    xq = ops.quantize_act(TQ6, to_dev(x, gpu))
    got = ops.mul_mat_wd_image(TQ6, img, xq, rows, cols, tokens, ops.mul_mat_work(rows, cols, tokens, TQ6, gpu))
    assert rel_l2(got.cpu().numpy(), oracle.matvec(TQ6, w, x)) < TOL


@pytest.mark.parametrize("rows,cols,tokens", [(5120, 17408, 8), (4096, 4096, 24), (130, 256, 1), (5120, 17408, 64),
                                              (2560, 9728, 48)])
def test_wd_image_model_shapes(gpu, oracle, rows, cols, tokens):
    """The config-5 down projection and other widths, through the split."""
    w = synth.make_weight(TQ6, rows, cols, seed=45, tag=rows)
    x = synth.make_act(cols, tokens, seed=45, tag=tokens)
    wd = to_dev(w, gpu)
    img = ops.wd_image(TQ6, wd, rows, cols)
    xq = ops.quantize_act(TQ6, to_dev(x, gpu))
    work = ops.mul_mat_work(rows, cols, tokens, TQ6, gpu)
    got = ops.mul_mat_wd_image(TQ6, img, xq, rows, cols, tokens, work)
    want = oracle.matvec(TQ6, w[: min(rows, 512)], x) if rows > 512 else oracle.matvec(TQ6, w, x)
    assert rel_l2(got.cpu().numpy()[:, : want.shape[1]], want) < TOL


@pytest.fixture()
def backend(gpu):
    be = ops.Backend(0)
    yield be
    be.close()


@pytest.mark.parametrize("tt,tokens", [(TQ6, 2), (TQ6, 3), (TQ6, 5), (TQ6, 8), (TQ6, 24), (TQ6, 32), (TQ6, 33),
                                       (TQ6, 64), (TQ6, 65),
                                       (po.TT_Q4_K, 2), (po.TT_Q4_K, 3), (po.TT_Q4_K, 8), (po.TT_Q4_K, 40),
                                       (po.TT_Q4_K, 130)])
def test_backend_batches_from_fragment_image(gpu, oracle, backend, tt, tokens):
    """matvecBatchK of a large Q6_K / Q4_K weight: the fragment image from 2
    tokens (Q6_K up to 64, then its plane image), built by prepare_linear;
    with images off the GGUF-row products, the same block integers."""
    rows, cols = 2048, 4608
    w = synth.make_weight(tt, rows, cols, seed=46, tag=tt)
    x = synth.make_act(cols, tokens, seed=46, tag=tokens)
    lin = backend.load_linear(tt, rows, cols, w)
    base = backend.mem_placed()
    assert backend.prepare_linear(lin) == 0
    img = rows * cols // 256 * (210 if tt == TQ6 else 144)  # the fragment image
    if tt == TQ6:
        img += _lib.load().qhip_mmq_image_bytes(tt, rows, cols)  # and the Q6_K plane image
    assert backend.mem_placed() - base >= img
    xd = to_dev(x, gpu)
    out = torch.empty((tokens, rows), device=gpu)
    backend.matvec_batch_k(out, lin, xd, tokens)
    backend.sync()
    got = out.cpu().numpy()
    assert rel_l2(got, oracle.matvec(tt, w, x)) < TOL
    backend.set_mmq_images(False)
    off = torch.empty((tokens, rows), device=gpu)
    backend.matvec_batch_k(off, lin, xd, tokens)
    backend.sync()
    # with the same slices in the same order (Q6_K 17..24 tokens, Q4_K from
    # 25) the GGUF-row kernel gives the same bits; elsewhere the same block
    # integers summed in another order
    if (tt == TQ6 and 17 <= tokens <= 24) or (tt == TQ4 and tokens > 24):
        assert np.array_equal(off.cpu().numpy(), got)
    else:
        assert rel_l2(off.cpu().numpy(), got) < 1e-6
    backend.set_mmq_images(True)




def wd_image_q4k_of(w, rows, cols):
    """The documented Q4_K fragment-image layout, from the GGUF bytes."""
    nsb = cols // 256
    ngrp = (rows + 31) // 32
    pad = np.zeros((ngrp * 32, nsb, 144), np.uint8)
    pad[:rows] = w.reshape(rows, nsb, 144)
    img = np.zeros((ngrp, nsb, 4608), np.uint8)
    g = pad.reshape(ngrp, 32, nsb, 144).transpose(0, 2, 1, 3)  # [group, sb, row, 144]
    for c in range(4):
        for k in range(2):
            img[:, :, 1024 * c + 512 * k:1024 * c + 512 * (k + 1)] = \
                g[:, :, :, 16 + 32 * c + 16 * k:32 + 32 * c + 16 * k].reshape(ngrp, nsb, 512)
    img[:, :, 4096:4608] = g[:, :, :, 0:16].reshape(ngrp, nsb, 512)
    return img.reshape(-1)


@pytest.mark.parametrize("rows,cols", [(1, 256), (31, 512), (32, 2304), (33, 256), (70, 1024)])
def test_wd_image_q4k_layout(gpu, rows, cols):
    w = synth.make_weight(TQ4, rows, cols, seed=50, tag=rows)
    n = ops.load().qhip_wd_image_bytes(TQ4, rows, cols)
    assert n == (rows + 31) // 32 * (cols // 256) * 4608
    img = ops.wd_image(TQ4, to_dev(w, gpu), rows, cols).cpu().numpy()
    assert np.array_equal(img[:n], wd_image_q4k_of(w, rows, cols))


@pytest.fixture(scope="module")
def q4(gpu):
    rows, cols = 333, 5120
    w = synth.make_weight(TQ4, rows, cols, seed=51, tag=TQ4)
    wd = to_dev(w, gpu)
    return rows, cols, w, wd, ops.wd_image(TQ4, wd, rows, cols)


@pytest.mark.parametrize("tokens", [1, 2, 8, 9, 24, 25, 32, 33, 64, 65, 96, 97, 130, 257])
def test_wd_image_q4k_vs_oracle(gpu, oracle, q4, tokens):
    """Every Q4_K launch from the image: above 24 tokens the same bits as from
    the GGUF rows (same slices, same order); up to 24 the K split inside the
    workgroup, the same block integers summed in another order."""
    rows, cols, w, wd, img = q4
    x = synth.make_act(cols, tokens, seed=52, tag=tokens)
    xq = ops.quantize_act(TQ4, to_dev(x, gpu))
    work = ops.mul_mat_work(rows, cols, tokens, TQ4, gpu)
    got = ops.mul_mat_wd_image(TQ4, img, xq, rows, cols, tokens, work)
    assert rel_l2(got.cpu().numpy(), oracle.matvec(TQ4, w, x)) < TOL
    assert torch.equal(got, ops.mul_mat_wd_image(TQ4, img, xq, rows, cols, tokens, work))
    raw = ops.mul_mat_split(TQ4, wd, xq, rows, cols, tokens, work, PATH_MMQ)
    if tokens > 24:
        assert torch.equal(got, raw)
    else:
        assert rel_l2(got.cpu().numpy(), raw.cpu().numpy()) < 1e-6
    plain = ops.mul_mat_wd_image(TQ4, img, xq, rows, cols, tokens)
    assert rel_l2(plain.cpu().numpy(), got.cpu().numpy()) < 1e-6


@pytest.mark.parametrize("tokens", [3, 20, 40, 72])
def test_wd_image_q4k_integers_exact(gpu, oracle, tokens):
    rows, cols = 96, 1024
    w = unit_scale_weight(TQ4, rows, cols, seed=53)
    x = unit_scale_act(cols, tokens, seed=53)
    act = oracle.quantize_act(TQ4, x)
    ints = oracle.block_ints(TQ4, w, act, cols).astype(np.int64)
    want = ints[:, :, 0::2].sum(-1) - ints[:, :, 1::2].sum(-1)
    assert np.abs(want).max() < 2 ** 24
    img = ops.wd_image(TQ4, to_dev(w, gpu), rows, cols)
    xq = ops.quantize_act(TQ4, to_dev(x, gpu))
    work = ops.mul_mat_work(rows, cols, tokens, TQ4, gpu)
    got = ops.mul_mat_wd_image(TQ4, img, xq, rows, cols, tokens, work).cpu().numpy()
    assert np.array_equal(got, want.astype(np.float32))


@pytest.mark.parametrize("tt,rows,cols,tokens", [(TQ6, 45, 256, 3), (TQ6, 97, 768, 16), (TQ4, 45, 256, 8),
                                                 (TQ4, 70, 1280, 24), (TQ6, 5120, 17408, 12), (TQ4, 17408, 5120, 20)])
def test_wd_image_k_split_in_workgroup(gpu, oracle, tt, rows, cols, tokens):
    """The in-workgroup K split: fewer super-blocks than waves (idle waves add
    zeros), row counts off the 32-row groups, the config-5 shapes; every
    rerun the same bits (the waves' sums are added in wave order)."""
    w = synth.make_weight(tt, rows, cols, seed=47, tag=rows)
    x = synth.make_act(cols, tokens, seed=47, tag=tokens)
    img = ops.wd_image(tt, to_dev(w, gpu), rows, cols)
    xq = ops.quantize_act(tt, to_dev(x, gpu))
    got = ops.mul_mat_wd_image(tt, img, xq, rows, cols, tokens)
    idx = np.arange(rows) if rows <= 512 else np.linspace(0, rows - 1, 512).astype(int)
    want = oracle.matvec(tt, np.ascontiguousarray(w[idx]), x)
    assert rel_l2(got.cpu().numpy()[:, idx], want) < TOL
    assert torch.equal(got, ops.mul_mat_wd_image(tt, img, xq, rows, cols, tokens))


# ---- Q8_0 fragment image --------------------------------------------------------
TQ8 = po.TT_Q8_0


def wd_image_q8_of(w, rows, cols):
    """The documented Q8_0 fragment-image layout, from the GGUF bytes."""
    nb = cols // 32
    ngrp = (rows + 31) // 32
    pad = np.zeros((ngrp * 32, nb, 34), np.uint8)
    pad[:rows] = w.reshape(rows, nb, 34)
    g = pad.reshape(ngrp, 32, nb, 34).transpose(0, 2, 1, 3)  # [group, block, row, 34]
    qs = np.zeros((ngrp, nb, 1024), np.uint8)
    for k in range(2):
        qs[:, :, 512 * k:512 * (k + 1)] = g[:, :, :, 2 + 16 * k:18 + 16 * k].reshape(ngrp, nb, 512)
    pos = [16 * ((i >> 2) & 1) + 4 * (i >> 3) + (i & 3) for i in range(32)]
    dd = np.zeros((ngrp, nb, 32, 2), np.uint8)
    dd[:, :, pos, :] = g[:, :, :, 0:2]
    return np.concatenate([qs.reshape(ngrp, -1), dd.reshape(ngrp, -1)], axis=1).reshape(-1)


@pytest.mark.parametrize("rows,cols", [(1, 256), (33, 512), (70, 1024), (64, 3584)])
def test_wd_image_q8_layout(gpu, rows, cols):
    w = synth.make_weight(TQ8, rows, cols, seed=60, tag=rows)
    n = ops.load().qhip_wd_image_bytes(TQ8, rows, cols)
    assert n == (rows + 31) // 32 * (cols // 32) * 1088
    img = ops.wd_image(TQ8, to_dev(w, gpu), rows, cols).cpu().numpy()
    assert np.array_equal(img[:n], wd_image_q8_of(w, rows, cols))


@pytest.mark.parametrize("rows,cols,tokens", [
    (100, 1024, 1), (100, 1024, 6), (100, 1024, 32), (100, 1024, 33), (100, 1024, 64), (100, 1024, 65),
    (100, 1024, 130), (33, 768, 40), (70, 256, 9), (64, 2048, 20), (96, 3584, 70), (40, 5120, 33)])
def test_wd_image_q8_vs_oracle(gpu, oracle, rows, cols, tokens):
    """The Q8_0 image MMQ at both token tiles, one and several 32-block
    super-chunks, partial ones (K not a multiple of 1024) and rows off the
    64-row tiles: within tolerance of the oracle, within 1e-6 of the MMQ on
    the GGUF rows (the same block integers scaled as (da sumi) dw and added
    in four K quarters), the same bits on every run."""
    w = synth.make_weight(TQ8, rows, cols, seed=61, tag=rows)
    x = synth.make_act(cols, tokens, seed=62, tag=tokens)
    wd = to_dev(w, gpu)
    img = ops.wd_image(TQ8, wd, rows, cols)
    xq = ops.quantize_act(TQ8, to_dev(x, gpu))
    got = ops.mul_mat_wd_image(TQ8, img, xq, rows, cols, tokens)
    assert rel_l2(got.cpu().numpy(), oracle.matvec(TQ8, w, x)) < TOL
    raw = ops.mul_mat(TQ8, wd, xq, rows, cols, tokens, PATH_MMQ)
    assert rel_l2(got.cpu().numpy(), raw.cpu().numpy()) < 1e-6
    assert torch.equal(got, ops.mul_mat_wd_image(TQ8, img, xq, rows, cols, tokens))


@pytest.mark.parametrize("cols,tokens", [(1024, 3), (1024, 40), (1024, 100), (2048, 33), (512, 64)])
def test_wd_image_q8_integers_exact(gpu, oracle, cols, tokens):
    """Unit scales: the exact sums of the block integers (up to 32 blocks of
    +-127 x +-127, so |sumi| reaches 2^19 where the MFMA's float bias trick
    must stay exact)."""
    rows = 96
    w = unit_scale_weight(TQ8, rows, cols, seed=63)
    x = unit_scale_act(cols, tokens, seed=63)
    act = oracle.quantize_act(TQ8, x)
    want = oracle.block_ints(TQ8, w, act, cols).astype(np.int64).sum(-1)
    assert np.abs(want).max() < 2 ** 24
    img = ops.wd_image(TQ8, to_dev(w, gpu), rows, cols)
    xq = ops.quantize_act(TQ8, to_dev(x, gpu))
    got = ops.mul_mat_wd_image(TQ8, img, xq, rows, cols, tokens).cpu().numpy()
    assert np.array_equal(got, want.astype(np.float32))


def test_wd_image_q8_extreme_blocks(gpu, oracle):
    """Every weight and activation value +-127 at unit scales: each block's
    |sumi| can reach 32 * 127 * 127, the bias trick's limit is 2^22."""
    rows, cols, tokens = 64, 1024, 48
    w = unit_scale_weight(TQ8, rows, cols, seed=64).reshape(rows, -1, 34)
    rng = np.random.default_rng(64)
    w[:, :, 2:] = np.where(rng.random((rows, w.shape[1], 32)) < 0.5, 0x81, 0x7F).astype(np.uint8)
    w[:8, :, 2:] = 0x7F  # rows of +127 only: against an all +-127 token, |sumi| = 32 * 127 * 127
    w = w.reshape(rows, -1)
    x = np.where(rng.random((tokens, cols)) < 0.5, -127.0, 127.0).astype(np.float32)
    x[0] = 127.0
    act = oracle.quantize_act(TQ8, x)
    want = oracle.block_ints(TQ8, w, act, cols).astype(np.int64).sum(-1)
    assert np.abs(want).max() == 32 * 32 * 127 * 127
    img = ops.wd_image(TQ8, to_dev(w, gpu), rows, cols)
    got = ops.mul_mat_wd_image(TQ8, img, ops.quantize_act(TQ8, to_dev(x, gpu)), rows, cols, tokens).cpu().numpy()
    assert np.array_equal(got, want.astype(np.float32))


@pytest.mark.parametrize("tokens", [512, 1673])
def test_wd_image_q8_config4(gpu, oracle, tokens):
    """Config 4's Q8_0 [3584, 1024] at the dense 512 tokens and the ragged
    batch's 1673 (packed by the ragged quantizer): 512 sampled rows against
    the oracle, all rows against the GGUF-row MMQ."""
    rows, cols = 3584, 1024
    w = synth.make_weight(TQ8, rows, cols, seed=65, tag=TQ8)
    wd = to_dev(w, gpu)
    img = ops.wd_image(TQ8, wd, rows, cols)
    if tokens == 512:
        x = synth.make_act(cols, tokens, seed=66, tag=tokens)
        xq = ops.quantize_act(TQ8, to_dev(x, gpu))
    else:
        lens = [int(v) for v in synth.ragged_lengths(8, 16, 256, seed=0)]
        assert sum(lens) == tokens
        seqs = [synth.make_act(cols, n, seed=67, tag=i) for i, n in enumerate(lens)]
        x = np.concatenate(seqs)
        xq, _, _ = ops.quantize_ragged(TQ8, [to_dev(s, gpu) for s in seqs], cols)
    got = ops.mul_mat_wd_image(TQ8, img, xq, rows, cols, tokens)
    idx = np.linspace(0, rows - 1, 512).astype(int)
    want = oracle.matvec(TQ8, np.ascontiguousarray(w[idx]), x)
    assert rel_l2(got.cpu().numpy()[:, idx], want) < TOL
    raw = ops.mul_mat(TQ8, wd, xq, rows, cols, tokens, PATH_MMQ)
    assert rel_l2(got.cpu().numpy(), raw.cpu().numpy()) < 1e-6


@pytest.mark.parametrize("rows,cols,tokens", [(3584, 1024, 6), (3584, 1024, 64), (6144, 1024, 200), (256, 2048, 64)])
def test_backend_batches_q8_from_fragment_image(gpu, oracle, backend, rows, cols, tokens):
    """matvecBatchK of a Q8_0 weight: from its fragment image from 6 tokens
    where K is at most 1024 (prepare_linear builds it), else the GGUF rows;
    with images off the GGUF-row products, within 1e-6."""
    w = synth.make_weight(TQ8, rows, cols, seed=68, tag=rows)
    x = synth.make_act(cols, tokens, seed=68, tag=tokens)
    lin = backend.load_linear(TQ8, rows, cols, w)
    base = backend.mem_placed()
    assert backend.prepare_linear(lin) == 0
    img = (rows + 31) // 32 * (cols // 32) * 1088
    assert (backend.mem_placed() - base >= img) == (cols <= 1024)
    xd = to_dev(x, gpu)
    out = torch.empty((tokens, rows), device=gpu)
    backend.matvec_batch_k(out, lin, xd, tokens)
    backend.sync()
    got = out.cpu().numpy()
    idx = np.arange(rows) if rows <= 512 else np.linspace(0, rows - 1, 512).astype(int)
    assert rel_l2(got[:, idx], oracle.matvec(TQ8, np.ascontiguousarray(w[idx]), x)) < TOL
    backend.set_mmq_images(False)
    off = torch.empty((tokens, rows), device=gpu)
    backend.matvec_batch_k(off, lin, xd, tokens)
    backend.sync()
    assert rel_l2(off.cpu().numpy(), got) < 1e-6
    backend.set_mmq_images(True)
