"""GPU: the K-quant GEMV image (Q4_K, Q6_K) -- its layout restated on the
host from the GGUF bytes, the image GEMV against the oracle and bit for bit
against the GGUF-layout GEMV of the same launch shape (every default shape:
team-of-lanes, whole-wave teams, several rows per team; the balanced teams
that only the Q6_K image takes at >= 4096 rows sum in another order), and
through the Exec
mirror, which reads a Q6_K weight's image where it quantizes separately:
bit-identical with images off, matvecPair over adjacent images, and no image
for the routes that keep the GGUF rows."""
import numpy as np
import pytest
import torch

import pyoracle as po
from qwen35_amd import ops, synth

TOL = 1e-5
KFORMATS = [po.TT_Q4_K, po.TT_Q6_K]
SB = {po.TT_Q4_K: 144, po.TT_Q6_K: 210}


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


def kimage_of(w, rows, cols, tt):
    """The documented layout: units in chunks of 64 (the last one m units),
    piece e of unit 64c + i at 16 (NP 64c + m e + i); then Q4_K's 16-byte
    super-block headers, or Q6_K's four scales per unit and f16 d per
    super-block."""
    U, S = cols // 64, cols // 256
    blk = w.reshape(rows, S, SB[tt])
    u = np.arange(U)
    sb, c, i = u // 4, u // 64, u % 64
    m = np.minimum(64, U - 64 * c)
    if tt == po.TT_Q4_K:
        q = u % 4
        pieces = [np.stack([blk[:, sb[k], 16 + 32 * q[k] + 16 * e:32 + 32 * q[k] + 16 * e] for k in range(U)], 1)
                  for e in range(2)]
        out = np.zeros((rows, 2 * U, 16), np.uint8)
        for e in range(2):
            out[:, 128 * c + m * e + i] = pieces[e]
        return np.concatenate([out.reshape(rows, -1), blk[:, :, 0:16].reshape(rows, -1)], axis=1)
    h, lh = (u // 2) % 2, u % 2
    offs = [64 * h + 16 * lh, 64 * h + 32 + 16 * lh, 128 + 32 * h + 16 * lh]
    out = np.zeros((rows, 3 * U, 16), np.uint8)
    for e in range(3):
        out[:, 192 * c + m * e + i] = np.stack([blk[:, sb[k], offs[e][k]:offs[e][k] + 16] for k in range(U)], 1)
    sc = np.stack([blk[:, sb[k], 192 + 8 * h[k] + lh[k] + np.array([0, 2, 4, 6])] for k in range(U)], 1)
    d = blk[:, :, 208:210]
    return np.concatenate([out.reshape(rows, -1), sc.reshape(rows, -1), d.reshape(rows, -1)], axis=1)


def test_kimage_layout_restatement_is_a_permutation():
    """Host-side check of the restatement itself: every GGUF byte lands once."""
    for tt, cols in ((po.TT_Q4_K, 2560), (po.TT_Q6_K, 9728), (po.TT_Q6_K, 2304)):
        rows = 2
        n = rows * (cols // 256) * SB[tt]
        w = (np.arange(n) % 251).astype(np.uint8)
        img = kimage_of(w, rows, cols, tt)
        assert img.shape == (rows, n // rows)
        assert np.array_equal(np.sort(img, axis=None), np.sort(w))


@pytest.mark.gpu
@pytest.mark.parametrize("tt", KFORMATS)
@pytest.mark.parametrize("rows,cols", [(1, 256), (3, 2560), (2, 4608), (2, 9728), (3, 2304), (1, 17408)])
def test_kimage_layout(gpu, tt, rows, cols):
    w = synth.make_weight(tt, rows, cols, seed=41, tag=tt)
    img = ops.gemv_image(tt, torch.from_numpy(w).to(gpu), rows, cols).cpu().numpy()
    assert np.array_equal(img[:rows * w.shape[1]].reshape(rows, -1), kimage_of(w, rows, cols, tt))


# (rows, cols, rows_per_lane): the default shapes (20- / 40-lane teams, 64
# lanes, two- and four-wave teams of 2 or 4 rows; Q6_K 20-lane teams of two
# rows at width 5120, Q4_K 64-lane teams of two rows at 4096; the Q6_K
# image's balanced teams from 4096 rows: one wave of two rows at widths 5120
# and 6144, four waves of two rows at 12288 and 13312 and of four at 17408
# and 20224 (a tail of 60 units per row: 240 of the team's 256 lanes), with a
# last team short of rows; width 7936, whose 60-unit tail does not fit one
# wave of two rows, keeps the default) and explicit row counts
KCASES = [(300, 2560, 0), (257, 1024, 0), (129, 5120, 0), (1, 2560, 0), (250, 2560, 1), (251, 2560, 2),
          (99, 4608, 0), (64, 9728, 0), (4100, 9728, 0), (77, 17408, 0), (40, 6144, 1), (33, 3840, 2),
          (4097, 2048, 0), (18, 2304, 0), (4100, 5120, 0), (4097, 4096, 0), (4099, 6144, 0),
          (4097, 12288, 0), (4099, 17408, 0), (4097, 13312, 0), (4096, 20224, 0), (4097, 7936, 0)]


def balanced(tt, rows, cols, nr):
    """Default-shape Q6_K image launches from 4096 rows of 64a + b units take
    the balanced teams (their own summation order): a = 1 with b <= 32, a = 3,
    a = 4 with b <= 64."""
    a, b = divmod(cols // 64, 64)
    return tt == po.TT_Q6_K and nr == 0 and rows >= 4096 and ((a == 1 and b <= 32) or a in (3, 4))


@pytest.mark.gpu
@pytest.mark.parametrize("tt", KFORMATS)
@pytest.mark.parametrize("rows,cols,nr", KCASES)
def test_kimage_gemv_vs_oracle_and_gguf(gpu, oracle, tt, rows, cols, nr):
    w = synth.make_weight(tt, rows, cols, seed=42, tag=tt)
    x = synth.make_act(cols, 1, seed=42)
    wd = torch.from_numpy(w).to(gpu)
    img = ops.gemv_image(tt, wd, rows, cols)
    xa = ops.quantize_act_image(tt, torch.from_numpy(x).to(gpu))
    xq = ops.quantize_act(tt, torch.from_numpy(x).to(gpu))
    assert torch.equal(xa[:xq.numel()], xq.reshape(-1))  # the reference Q8_K rows
    out = ops.mul_mat_vec_image(tt, img, xa, rows, cols, nr).cpu().numpy()
    assert rel_l2(out, oracle.matvec(tt, w, x)[0]) < TOL
    # the GGUF-layout GEMV of the same shape: same units, same order (the
    # balanced teams: the same block integers, summed in another order)
    if (rows * w.shape[1]) % 4 == 0:
        raw = ops.gemv_tuned(tt, wd, xq, rows, cols, 1, 0, 0, rows_per_lane=nr).cpu().numpy().reshape(-1)
        if balanced(tt, rows, cols, nr):
            assert rel_l2(out, raw) < 1e-6
        else:
            assert np.array_equal(out, raw)


@pytest.mark.gpu
@pytest.mark.parametrize("tt", KFORMATS)
def test_kimage_gemv_integers_exact(gpu, oracle, tt):
    """d = dmin = 1 and activations of Q8_K scale 1: each output is the exact
    integer of its row (Q4_K isum - summs, Q6_K the scaled sum)."""
    from test_gpu_mmq import unit_scale_act, unit_scale_weight
    rows, cols = 96, 2560
    w = unit_scale_weight(tt, rows, cols, seed=43)
    x = unit_scale_act(cols, 1, seed=43)
    act = oracle.quantize_act(tt, x)
    ints = oracle.block_ints(tt, w, act, cols).astype(np.int64)
    want = ints[:, :, 0::2].sum(-1) - ints[:, :, 1::2].sum(-1) if tt == po.TT_Q4_K else ints.sum(-1)
    assert np.abs(want).max() < 2 ** 24
    img = ops.gemv_image(tt, torch.from_numpy(w).to(gpu), rows, cols)
    xa = ops.quantize_act_image(tt, torch.from_numpy(x).to(gpu))
    for nr in (0, 1, 2):
        out = ops.mul_mat_vec_image(tt, img, xa, rows, cols, nr).cpu().numpy()
        assert np.array_equal(out, want[0].astype(np.float32))


@pytest.fixture()
def backend(gpu):
    be = ops.Backend(0)
    yield be
    be.close()


# the mirror's separate quantize + GEMV routes of Q6_K: every width past the
# one-launch form's (up to 4096; long rows included, in place of the split-K
# form), and rows past the one-launch form's 32768
MIRROR = [(po.TT_Q6_K, 1500, 5120), (po.TT_Q6_K, 700, 6144), (po.TT_Q6_K, 40000, 1024),
          (po.TT_Q6_K, 2560, 9728), (po.TT_Q6_K, 1000, 17408), (po.TT_Q6_K, 4100, 6144)]
# routes that keep the GGUF rows: the one-launch form, Q4_K
NO_IMAGE = [(po.TT_Q6_K, 700, 4096), (po.TT_Q4_K, 1500, 5120), (po.TT_Q4_K, 9728, 2560)]


@pytest.mark.gpu
@pytest.mark.parametrize("tt,rows,cols", MIRROR)
def test_backend_matvec_reads_kimage(gpu, oracle, backend, tt, rows, cols):
    w = synth.make_weight(tt, rows, cols, seed=44, tag=tt)
    x = synth.make_act(cols, 1, seed=44)
    lin = backend.load_linear(tt, rows, cols, w)
    before = backend.mem_placed()
    assert backend.prepare_linear(lin) == 0
    assert backend.mem_placed() - before >= rows * w.shape[1]  # the image
    xd = torch.from_numpy(x[0]).to(gpu)
    out = torch.empty(rows, device=gpu)
    backend.matvec(out, lin, xd)
    backend.sync()
    got = out.cpu().numpy()
    assert rel_l2(got, oracle.matvec(tt, w, x)[0]) < TOL
    # images off: the GGUF rows -- through the same launch (the same bits)
    # where the mirror would quantize separately anyway, through the split-K
    # one-launch form (the same block integers, summed in another order) on
    # rows of 8192 values and more, and in another order too where the image
    # takes the balanced teams
    backend.set_gemv_images(False)
    out2 = torch.empty(rows, device=gpu)
    backend.matvec(out2, lin, xd)
    backend.sync()
    backend.set_gemv_images(True)
    if cols >= 8192 or balanced(tt, rows, cols, 0):
        assert rel_l2(out2.cpu().numpy(), got) < 1e-6
    else:
        assert np.array_equal(out2.cpu().numpy(), got)


@pytest.mark.gpu
@pytest.mark.parametrize("tt,rows,cols", NO_IMAGE)
def test_backend_no_kimage_where_gguf_rows_win(gpu, oracle, backend, tt, rows, cols):
    w = synth.make_weight(tt, rows, cols, seed=46, tag=tt)
    x = synth.make_act(cols, 1, seed=46)
    lin = backend.load_linear(tt, rows, cols, w)
    # the prefill images first (GEMV images off), then whatever images on adds
    backend.set_gemv_images(False)
    assert backend.prepare_linear(lin) == 0
    before = backend.mem_placed()
    backend.set_gemv_images(True)
    assert backend.prepare_linear(lin) == 0
    assert backend.mem_placed() == before  # no GEMV image built
    out = torch.empty(rows, device=gpu)
    backend.matvec(out, lin, torch.from_numpy(x[0]).to(gpu))
    backend.sync()
    assert rel_l2(out.cpu().numpy(), oracle.matvec(tt, w, x)[0]) < TOL


@pytest.mark.gpu
def test_backend_kimage_pair_and_memo(gpu, oracle, backend):
    """matvecPair over the adjacent Q6_K images of gate and up, then the
    second weight alone from inside them, with the activation memo on."""
    tt, rows, cols = po.TT_Q6_K, 1500, 5120
    wa = synth.make_weight(tt, rows, cols, seed=45, tag=1)
    wb = synth.make_weight(tt, rows, cols, seed=45, tag=2)
    x = synth.make_act(cols, 1, seed=45)
    la = backend.load_linear(tt, rows, cols, wa)
    lb = backend.load_linear(tt, rows, cols, wb)
    backend.prepare_linear(la)
    backend.prepare_linear(lb)
    backend.set_act_memo(True)
    backend.step_begin(0)
    xd = torch.from_numpy(x[0]).to(gpu)
    out = torch.empty(2 * rows, device=gpu)
    backend.matvec_pair(out, la, lb, xd)
    ob = torch.empty(rows, device=gpu)
    backend.matvec(ob, lb, xd)
    backend.sync()
    got = out.cpu().numpy()
    assert rel_l2(got[:rows], oracle.matvec(tt, wa, x)[0]) < TOL
    assert rel_l2(got[rows:], oracle.matvec(tt, wb, x)[0]) < TOL
    # the single weight takes its own launch shape (rows per team may differ)
    assert rel_l2(ob.cpu().numpy(), got[rows:]) < 1e-6
    backend.set_act_memo(False)
