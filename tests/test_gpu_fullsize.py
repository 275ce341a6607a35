"""GPU parity at the BASELINE sizes of the prefill configurations, through the
C ABI: config 4 dense (Q8_0 [3584, 1024], 512 tokens) and config 5 (Q4_K
[17408, 5120] and Q6_K [5120, 17408] at 4, 16, 64 and 512 tokens), on every
kernel those shapes reach: the automatic path with the split-K workspace the
Exec mirror passes (split MMQ tiles for small grids, the weights-direct Q4_K
kernel from 128 tokens, the GEMV below the crossover), the explicit tile MMQ,
the Q6_K weight image, and the Exec mirror's matvecBatchK.

Bar: float outputs within 1e-5 relative L2 of the oracle on 512 sampled rows
(every token, so every token tile is covered); with unit scales the float
result is the sum of the per-block integers and must equal the oracle's
integers exactly, at full K; a split-K launch returns the same bits on every
run (the slices are added in slice order).
"""
import numpy as np
import pytest
import torch

import pyoracle as po
from qwen35_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu

TOL = 1e-5
NSAMPLE = 512
PATH_AUTO, PATH_GEMV, PATH_MMQ = 0, 1, 2
F16_ONE = np.array([0x00, 0x3C], np.uint8)
THREADS = 16  # the GPU box's CPU share


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def sample_rows(rows, seed):
    rng = np.random.default_rng(seed)
    idx = rng.choice(rows, NSAMPLE - 2, replace=False)
    return np.unique(np.concatenate([[0, rows - 1], idx]))


_W = {}


def weight(tt, rows, cols):
    key = (tt, rows, cols)
    if key not in _W:
        _W.clear()
        _W[key] = synth.make_weight(tt, rows, cols, seed=0, tag=tt)
    return _W[key]


def check(got, want, what):
    r = rel_l2(got, want)
    assert np.all(np.isfinite(got)), what
    assert r < TOL, (what, r)


def test_cfg4_dense_512(gpu, oracle):
    tt, rows, cols, T = po.TT_Q8_0, 3584, 1024, 512
    print(f"cfg4 dense Q8_0 [{rows}x{cols}] T={T}", flush=True)
    w = weight(tt, rows, cols)
    x = synth.make_act(cols, T, seed=400)
    idx = sample_rows(rows, 4)
    want = oracle.matvec(tt, np.ascontiguousarray(w[idx]), x, nthreads=THREADS)
    wd = to_dev(w, gpu)
    xq = ops.quantize_act(tt, to_dev(x, gpu))
    work = ops.mul_mat_work(rows, cols, T, tt, gpu)
    for path in (PATH_AUTO, PATH_MMQ):
        got = ops.mul_mat_split(tt, wd, xq, rows, cols, T, work, path).cpu().numpy()
        check(got[:, idx], want, f"path {path}")
    got = ops.mul_mat(tt, wd, xq, rows, cols, T).cpu().numpy()
    check(got[:, idx], want, "qhip_launch_mul_mat_vec")


CFG5 = [(po.TT_Q4_K, 17408, 5120), (po.TT_Q6_K, 5120, 17408)]


@pytest.mark.parametrize("T", [4, 16, 64, 512])
@pytest.mark.parametrize("tt,rows,cols", CFG5, ids=["Q4_K-17408x5120", "Q6_K-5120x17408"])
def test_cfg5_every_path(gpu, oracle, tt, rows, cols, T):
    print(f"cfg5 {po.NAMES[tt]} [{rows}x{cols}] T={T}", flush=True)
    w = weight(tt, rows, cols)
    x = synth.make_act(cols, T, seed=500 + T)
    idx = sample_rows(rows, T)
    want = oracle.matvec(tt, np.ascontiguousarray(w[idx]), x, nthreads=THREADS)
    wd = to_dev(w, gpu)
    xq = ops.quantize_act(tt, to_dev(x, gpu))
    work = ops.mul_mat_work(rows, cols, T, tt, gpu)
    # the automatic path with and without the split-K workspace, the GEMV, the tile MMQ
    for name, fn in (("auto+work", lambda: ops.mul_mat_split(tt, wd, xq, rows, cols, T, work, PATH_AUTO)),
                     ("auto", lambda: ops.mul_mat(tt, wd, xq, rows, cols, T)),
                     ("gemv", lambda: ops.mul_mat(tt, wd, xq, rows, cols, T, PATH_GEMV)),
                     ("mmq+work", lambda: ops.mul_mat_split(tt, wd, xq, rows, cols, T, work, PATH_MMQ)),
                     ("mmq", lambda: ops.mul_mat(tt, wd, xq, rows, cols, T, PATH_MMQ))):
        check(fn().cpu().numpy()[:, idx], want, name)
    if tt == po.TT_Q6_K:
        img = ops.mmq_image(tt, wd, rows, cols)
        check(ops.mul_mat_image(tt, img, xq, rows, cols, T, work=work).cpu().numpy()[:, idx], want, "image+work")
        check(ops.mul_mat_image(tt, img, xq, rows, cols, T).cpu().numpy()[:, idx], want, "image")
        del img
    # the Exec mirror's matvecBatchK (Q6_K: from its image, built on first use)
    be = ops.Backend(0)
    try:
        lin = be.wrap_linear(tt, rows, cols, wd)
        out = torch.empty((T, rows), device=gpu)
        be.matvec_batch_k(out, lin, to_dev(x, gpu), T)
        be.sync()
        check(out.cpu().numpy()[:, idx], want, "backend")
        be.free_linear(lin)
    finally:
        be.close()


def _unit_q4k(w):
    blk = w.reshape(w.shape[0], -1, 144)
    blk[:, :, 0:2] = F16_ONE
    blk[:, :, 2:4] = F16_ONE
    return w


def _unit_q6k(w):
    w.reshape(w.shape[0], -1, 210)[:, :, 208:210] = F16_ONE
    return w


def _unit_act(cols, tokens, seed):
    # small integers with one +-127 per 256 values: the Q8_K scale is exactly
    # 1.0, the quantized values equal x, and the sums over 17408 values stay
    # far below 2^24
    rng = np.random.default_rng(seed)
    x = rng.integers(-8, 9, (tokens, cols)).astype(np.float32)
    x[:, ::256] = np.where(rng.random((tokens, cols // 256)) < 0.5, -127.0, 127.0)
    return x


@pytest.mark.parametrize("T", [64, 512])
@pytest.mark.parametrize("tt,rows,cols", CFG5, ids=["Q4_K-17408x5120", "Q6_K-5120x17408"])
def test_cfg5_block_integers_exact_full_k(gpu, oracle, tt, rows, cols, T):
    """Unit scales at full K: every float the MMQ adds is an integer below
    2^24, so the output must equal the oracle's block-integer sums exactly
    (split slices included: any sum of consecutive super-blocks stays below
    2^24 when every prefix does, by half)."""
    print(f"cfg5 unit-scale {po.NAMES[tt]} [{rows}x{cols}] T={T}", flush=True)
    w = weight(tt, rows, cols).copy()
    w = _unit_q4k(w) if tt == po.TT_Q4_K else _unit_q6k(w)
    x = _unit_act(cols, T, seed=T)
    act = oracle.quantize_act(tt, x)
    idx = sample_rows(rows, 7 + T)[:: 4]  # 128 rows: block_ints walks them one by one
    ints = oracle.block_ints(tt, np.ascontiguousarray(w[idx]), act, cols).astype(np.int64)
    if tt == po.TT_Q4_K:
        per_sb = ints[:, :, 0::2] - ints[:, :, 1::2]  # isum - summs per super-block
    else:
        per_sb = ints
    assert np.abs(np.cumsum(per_sb, axis=-1)).max() < 2 ** 23
    want = per_sb.sum(-1)
    wd = to_dev(w, gpu)
    xq = ops.quantize_act(tt, to_dev(x, gpu))
    assert np.array_equal(xq.cpu().numpy(), act)
    work = ops.mul_mat_work(rows, cols, T, tt, gpu)
    outs = {"auto+work": ops.mul_mat_split(tt, wd, xq, rows, cols, T, work, PATH_AUTO),
            "mmq": ops.mul_mat(tt, wd, xq, rows, cols, T, PATH_MMQ)}
    if tt == po.TT_Q6_K:
        img = ops.mmq_image(tt, wd, rows, cols)
        outs["image+work"] = ops.mul_mat_image(tt, img, xq, rows, cols, T, work=work)
    for name, o in outs.items():
        got = o.cpu().numpy()[:, idx]
        assert np.array_equal(got, want.astype(np.float32)), name


@pytest.mark.parametrize("tt,rows,cols", CFG5, ids=["Q4_K-17408x5120", "Q6_K-5120x17408"])
def test_split_k_is_deterministic(gpu, oracle, tt, rows, cols):
    """The split launches (cfg5 at 16 tokens: 136 / 40 row tiles, K cut into
    slices) return the same bits on every run, and agree with the unsplit
    launch within the tolerance."""
    T = 16
    w = weight(tt, rows, cols)
    x = synth.make_act(cols, T, seed=77)
    wd = to_dev(w, gpu)
    xq = ops.quantize_act(tt, to_dev(x, gpu))
    work = ops.mul_mat_work(rows, cols, T, tt, gpu)
    assert work is not None  # this shape splits
    runs = [ops.mul_mat_split(tt, wd, xq, rows, cols, T, work, PATH_MMQ).cpu().numpy() for _ in range(3)]
    for r in runs[1:]:
        assert np.array_equal(r.view(np.uint32), runs[0].view(np.uint32))
    unsplit = ops.mul_mat(tt, wd, xq, rows, cols, T, PATH_MMQ).cpu().numpy()
    assert rel_l2(runs[0], unsplit) < TOL
    if tt == po.TT_Q6_K:
        img = ops.mmq_image(tt, wd, rows, cols)
        ri = [ops.mul_mat_image(tt, img, xq, rows, cols, T, work=work).cpu().numpy() for _ in range(3)]
        for r in ri[1:]:
            assert np.array_equal(r.view(np.uint32), ri[0].view(np.uint32))
        assert rel_l2(ri[0], unsplit) < TOL
    idx = sample_rows(rows, 9)
    want = oracle.matvec(tt, np.ascontiguousarray(w[idx]), x, nthreads=THREADS)
    check(runs[0][:, idx], want, "split")


def test_backend_image_budget_and_opt_out(gpu, oracle):
    """A backend whose device budget cannot hold the Q6_K image, or with
    images off, runs the tile MMQ on the GGUF bytes: same parity, no image
    placed; prepare_linear builds the image at load time when it fits."""
    tt, rows, cols, T = po.TT_Q6_K, 4096, 4608, 128  # a prefill long enough for the image path
    w = synth.make_weight(tt, rows, cols, seed=3, tag=tt)
    x = synth.make_act(cols, T, seed=3)
    want = oracle.matvec(tt, w, x, nthreads=THREADS)
    img_bytes = _lib.load().qhip_mmq_image_bytes(tt, rows, cols)  # the plane image, 2.5x the GGUF bytes
    frag_bytes = rows * cols // 256 * 210  # the few-token fragment image, built with it
    gemv_bytes = rows * cols // 256 * 210  # and the decode matvec's GEMV image at this width
    xd = to_dev(x, gpu)
    for mode in ("capped", "off", "prepared"):
        be = ops.Backend(0)
        try:
            lin = be.load_linear(tt, rows, cols, w)
            base = be.mem_placed()
            if mode == "capped":
                be.set_mem_budget(base + (20 << 20))  # scratch and workspace fit, the 39 MB image does not
            elif mode == "off":
                be.set_mmq_images(False)
            else:
                assert be.prepare_linear(lin) == 0
                assert be.mem_placed() == base + img_bytes + frag_bytes + gemv_bytes
            out = torch.empty((T, rows), device=gpu)
            for rep in range(2):
                be.matvec_batch_k(out, lin, xd, T)
                be.sync()
                check(out.cpu().numpy(), want, f"{mode} rep {rep}")
            placed_img = be.mem_placed() - base
            if mode == "prepared":
                assert placed_img >= img_bytes
            else:
                assert placed_img < img_bytes, mode  # scratch and workspace only
            if mode == "capped":
                assert be.prepare_linear(lin) == -1  # declined: past the budget
        finally:
            be.close()


def test_backend_wrapped_memory_reused_after_free(gpu, oracle):
    """wrap_linear + free_linear, then another weight of the same shape in the
    same device memory: the second prefill must not meet the first weight's
    image."""
    tt, rows, cols, T = po.TT_Q6_K, 256, 2304, 128  # long enough for the image path
    wa = synth.make_weight(tt, rows, cols, seed=11, tag=tt)
    wb = synth.make_weight(tt, rows, cols, seed=12, tag=tt)
    x = synth.make_act(cols, T, seed=11)
    xd = to_dev(x, gpu)
    mem = to_dev(wa, gpu)
    be = ops.Backend(0)
    try:
        out = torch.empty((T, rows), device=gpu)
        lin = be.wrap_linear(tt, rows, cols, mem)
        be.matvec_batch_k(out, lin, xd, T)
        be.sync()
        check(out.cpu().numpy(), oracle.matvec(tt, wa, x), "first weight")
        be.free_linear(lin)
        mem.copy_(to_dev(wb, gpu))
        lin = be.wrap_linear(tt, rows, cols, mem)
        be.matvec_batch_k(out, lin, xd, T)
        be.sync()
        check(out.cpu().numpy(), oracle.matvec(tt, wb, x), "second weight, same memory")
    finally:
        be.close()


def test_budget_rejects_upload(gpu):
    be = ops.Backend(0)
    try:
        be.set_mem_budget(1 << 20)
        w = synth.make_weight(po.TT_Q8_0, 64, 32768, seed=1, tag=8)  # 2.2 MB
        with pytest.raises(Exception):
            be.load_linear(po.TT_Q8_0, 64, 32768, w)
        assert be.mem_placed() == 0
    finally:
        be.close()


def test_q6k_plane_image_whole_and_sliced_tiles(gpu, oracle):
    """The Q6_K plane-image MMQ on a grid with more tiles than resident
    workgroups: whole tiles, then the remaining tiles cut over K (with the
    workspace) or whole again (without); both within the tolerance on the
    sampled rows (the last row tile is partly past the end), the split form
    bit-equal on a rerun."""
    tt, rows, cols, T = po.TT_Q6_K, 16480, 2304, 512
    w = synth.make_weight(tt, rows, cols, seed=21, tag=tt)
    x = synth.make_act(cols, T, seed=21)
    idx = sample_rows(rows, 21)
    idx = np.unique(np.concatenate([idx, np.arange(rows - 96, rows)]))
    want = oracle.matvec(tt, np.ascontiguousarray(w[idx]), x, nthreads=THREADS)
    wd = to_dev(w, gpu)
    xq = ops.quantize_act(tt, to_dev(x, gpu))
    img = ops.mmq_image(tt, wd, rows, cols)
    del wd
    work = ops.mul_mat_work(rows, cols, T, tt, gpu)
    assert work is not None
    a = ops.mul_mat_image(tt, img, xq, rows, cols, T, work=work)
    check(a.cpu().numpy()[:, idx], want, "image+work")
    assert torch.equal(a, ops.mul_mat_image(tt, img, xq, rows, cols, T, work=work))
    check(ops.mul_mat_image(tt, img, xq, rows, cols, T).cpu().numpy()[:, idx], want, "image")


@pytest.mark.parametrize("rows,cols", [(17408, 5120), (16480, 2304)], ids=["17408x5120", "16480x2304"])
def test_q4k_weights_direct_whole_and_sliced_tiles(gpu, oracle, rows, cols):
    """The Q4_K weights-direct MMQ at 512 tokens, more tiles than resident
    workgroups: the whole rounds of tiles run over all of K and only the
    tiles of the last, partial round are cut into K slices (with the
    workspace; without it every tile is whole).  From the GGUF rows and from
    the fragment image: within the tolerance on the sampled rows plus the
    last two row tiles (the sliced ones; at 16480 rows the last is partly
    past the end), bit-equal on a rerun, and within the tolerance of the
    unsplit launch over the whole output."""
    tt, T = po.TT_Q4_K, 512
    print(f"Q4_K weights-direct whole+sliced [{rows}x{cols}] T={T}", flush=True)
    w = synth.make_weight(tt, rows, cols, seed=31, tag=tt)
    x = synth.make_act(cols, T, seed=31)
    idx = sample_rows(rows, 31)
    idx = np.unique(np.concatenate([idx, np.arange(rows - 192, rows)]))
    want = oracle.matvec(tt, np.ascontiguousarray(w[idx]), x, nthreads=THREADS)
    wd = to_dev(w, gpu)
    xq = ops.quantize_act(tt, to_dev(x, gpu))
    work = ops.mul_mat_work(rows, cols, T, tt, gpu)
    assert work is not None  # the last round is sliced
    a = ops.mul_mat_split(tt, wd, xq, rows, cols, T, work, PATH_MMQ)
    check(a.cpu().numpy()[:, idx], want, "gguf+work")
    assert torch.equal(a, ops.mul_mat_split(tt, wd, xq, rows, cols, T, work, PATH_MMQ))
    whole = ops.mul_mat(tt, wd, xq, rows, cols, T, PATH_MMQ)
    assert rel_l2(a.cpu().numpy(), whole.cpu().numpy()) < TOL
    img = ops.wd_image(tt, wd, rows, cols)
    b = ops.mul_mat_wd_image(tt, img, xq, rows, cols, T, work)
    check(b.cpu().numpy()[:, idx], want, "image+work")
    assert torch.equal(b, ops.mul_mat_wd_image(tt, img, xq, rows, cols, T, work))
    check(ops.mul_mat_wd_image(tt, img, xq, rows, cols, T).cpu().numpy()[:, idx], want, "image")
