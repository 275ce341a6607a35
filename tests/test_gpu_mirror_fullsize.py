"""GPU: the Exec mirror's batch-1 routes at their full BASELINE sizes, through
`qhip_backend_matvec` -- the launches the headline bench times and an engine's
decode step runs:

* config 3, IQ4_NL [248320, 2560]: the split quantize + GEMV-image launch
  (`k_gemv_img`, image built by prepare_linear), 10,347 workgroups;
* config 5 Q6_K [5120, 17408] (down projection) and Q6_K [4096, 12288]: the
  quantize launch, then the balanced GEMV (`k_gemv_bal`: four-wave teams of
  four rows at 17408 values, of two rows at 12288, every load of a lane at
  once) from the weight's K-quant image, built by prepare_linear;
* config 5 Q4_K [17408, 5120]: quantize + the multi-wave GEMV.

Bar: the float outputs within 1e-5 relative L2 of the oracle on 512 sampled
rows plus the whole last row tile; the mirror's output bit-equal to the
explicit C-ABI launch of the route it is documented to take (which pins the
route and its default launch shape); and, with unit scales, every row of the
full output equal to the oracle's exact integer sum.

Unit-scale bounds (every partial sum the GPU forms is a sum of a subset of the
per-block terms, so it is exact when the sum of their magnitudes is below
2^24): activations are integers in [-8, 8] with one +-127 per activation
block, so the activation scale is exactly 1.0 and the quantized values equal
x.  IQ4_NL (d = 1): |sumi| <= 31*127*8 + 127*127 per 32-value block, 80
blocks: 3.8e6.  Q6_K (d = 1, sub-block scales +-1): <= 16*(15*32*8 + 32*127)
per super-block, 68 super-blocks: 8.6e6.  Q4_K (d = dmin = 1, every scale
byte 0x01, i.e. sub-block scales 1, mins 1 / 0): <= 256*15*8 + 8*15*127 + the
mins term per super-block, 20 super-blocks: 1.0e6.
"""
import numpy as np
import pytest
import torch

import pyoracle as po
from qwen35_amd import ops, synth

pytestmark = pytest.mark.gpu

TOL = 1e-5
NSAMPLE = 512
THREADS = 16  # the GPU box's CPU share
F16_ONE = np.array([0x00, 0x3C], np.uint8)


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def sampled_rows(rows, seed, tail=64):
    rng = np.random.default_rng(seed)
    idx = rng.choice(rows, NSAMPLE, replace=False)
    return np.unique(np.concatenate([idx, np.arange(rows - tail, rows)]))


def unit_weight(tt, w, seed):
    w = w.copy()
    if tt == po.TT_IQ4_NL:
        w.reshape(w.shape[0], -1, 18)[:, :, 0:2] = F16_ONE
    elif tt == po.TT_Q6_K:
        blk = w.reshape(w.shape[0], -1, 210)
        blk[:, :, 208:210] = F16_ONE
        rng = np.random.default_rng(seed)
        blk[:, :, 192:208] = np.where(rng.random(blk[:, :, 192:208].shape) < 0.5, 0x01, 0xFF).astype(np.uint8)
    elif tt == po.TT_Q4_K:
        blk = w.reshape(w.shape[0], -1, 144)
        blk[:, :, 0:2] = F16_ONE
        blk[:, :, 2:4] = F16_ONE
        blk[:, :, 4:16] = 0x01
    else:
        raise ValueError(tt)
    return w


def unit_act(tt, cols, seed):
    rng = np.random.default_rng(seed)
    x = rng.integers(-8, 9, (1, cols)).astype(np.float32)
    step = po.act_block_elems(tt)
    x[:, ::step] = np.where(rng.random((1, cols // step)) < 0.5, -127.0, 127.0)
    return x


def explicit_route(tt, wd, xd, rows, cols, gpu):
    """The C-ABI launch the mirror's batch-1 matvec is documented to take at this shape."""
    if tt == po.TT_IQ4_NL:
        img = ops.gemv_image(tt, wd, rows, cols)
        return ops.mul_mat_vec_image(tt, img, ops.quantize_act_image(tt, xd[None, :]), rows, cols)
    if tt == po.TT_Q6_K:
        # the K-quant image GEMV at its default launch shape (the balanced
        # teams at these widths)
        img = ops.gemv_image(tt, wd, rows, cols)
        return ops.mul_mat_vec_image(tt, img, ops.quantize_act_image(tt, xd[None, :]), rows, cols)
    xq = ops.quantize_act(tt, xd[None, :])
    return ops.mul_mat(tt, wd, xq, rows, cols, 1, 1)[0]


ROUTES = [("cfg3-iq4_nl-image", po.TT_IQ4_NL, 248320, 2560),
          ("cfg5-q6_k-kimage", po.TT_Q6_K, 5120, 17408),
          ("q6_k-kimage-12288", po.TT_Q6_K, 4096, 12288),
          ("cfg5-q4_k-gemv", po.TT_Q4_K, 17408, 5120)]


@pytest.mark.parametrize("name,tt,rows,cols", ROUTES, ids=[r[0] for r in ROUTES])
def test_mirror_matvec_full_size(gpu, oracle, name, tt, rows, cols):
    print(f"mirror matvec {name} [{rows}x{cols}]", flush=True)
    w = synth.make_weight(tt, rows, cols, seed=0, tag=tt)
    x = synth.make_act(cols, 1, seed=3)
    idx = sampled_rows(rows, rows + cols)
    want = oracle.matvec(tt, np.ascontiguousarray(w[idx]), x, nthreads=THREADS)[0]
    be = ops.Backend(0)
    try:
        lin = be.load_linear(tt, rows, cols, w)
        base = be.mem_placed()
        be.prepare_linear(lin)
        if tt == po.TT_IQ4_NL:
            # the GEMV image is built, as many bytes again as the GGUF rows
            n = be.lib.qhip_gemv_image_bytes(tt, rows, cols)
            assert n >= rows * w.shape[1]
            assert be.mem_placed() - base == (n + 255) // 256 * 256
        xd = to_dev(x[0], gpu)
        out = torch.empty(rows, device=gpu)
        be.matvec(out, lin, xd)
        be.sync()
        got = out.cpu().numpy()
        assert np.all(np.isfinite(got))
        assert rel_l2(got[idx], want) < TOL, rel_l2(got[idx], want)
        # the route and its launch shape: the explicit launch gives the same bits
        wd = to_dev(w, gpu)
        ref = explicit_route(tt, wd, xd, rows, cols, gpu).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
        # a second call on the same backend (split-K counters back at zero)
        out2 = torch.empty(rows, device=gpu)
        be.matvec(out2, lin, xd)
        be.sync()
        assert torch.equal(out, out2)
    finally:
        be.close()


@pytest.mark.parametrize("name,tt,rows,cols", ROUTES, ids=[r[0] for r in ROUTES])
def test_mirror_matvec_full_size_exact_integers(gpu, oracle, name, tt, rows, cols):
    """Unit scales: every row of the full output is the exact integer sum."""
    print(f"mirror matvec unit-scale {name} [{rows}x{cols}]", flush=True)
    w = unit_weight(tt, synth.make_weight(tt, rows, cols, seed=1, tag=tt), seed=rows)
    x = unit_act(tt, cols, seed=cols)
    act = oracle.quantize_act(tt, x)
    # the activation scale is 1.0 and the quantized values equal x
    if po.act_block_elems(tt) == 32:
        blk = act.reshape(-1, 34)
        assert np.all(blk[:, 0:2] == F16_ONE)
        assert np.array_equal(blk[:, 2:].view(np.int8).reshape(-1), x[0].astype(np.int8))
    else:
        blk = act.reshape(-1, 292)
        assert np.all(blk[:, 0:4].copy().view(np.float32) == 1.0)
        assert np.array_equal(blk[:, 4:260].copy().view(np.int8).reshape(-1), x[0].astype(np.int8))
    want = oracle.matvec(tt, w, x, nthreads=THREADS)[0]
    assert np.array_equal(want, np.round(want))
    # the oracle's sum is the sum of its own per-block integers on sampled rows
    idx = sampled_rows(rows, 5, tail=8)[::8]
    ints = oracle.block_ints(tt, np.ascontiguousarray(w[idx]), act, cols)[0].astype(np.int64)
    per_row = ints[:, 0::2].sum(-1) - ints[:, 1::2].sum(-1) if tt == po.TT_Q4_K else ints.sum(-1)
    assert np.array_equal(per_row.astype(np.float32), want[idx])
    be = ops.Backend(0)
    try:
        lin = be.load_linear(tt, rows, cols, w)
        be.prepare_linear(lin)
        out = torch.empty(rows, device=gpu)
        be.matvec(out, lin, to_dev(x[0], gpu))
        be.sync()
        got = out.cpu().numpy()
        bad = np.flatnonzero(got != want)
        assert bad.size == 0, (bad[:8], got[bad[:8]], want[bad[:8]])
    finally:
        be.close()
