"""GPU: the GEMV weight image of the 32-value formats (IQ4_NL, Q4_0, Q8_0) --
the image and split-activation layouts, the image GEMV against the oracle
(every launch shape, odd row counts, exact integers at unit scales) and
through the Exec mirror (image built and found, matvecPair over adjacent
images, the activation memo across layouts, free_linear on reused memory)."""
import numpy as np
import pytest
import torch

import pyoracle as po
from qwen35_amd import ops, synth

pytestmark = pytest.mark.gpu
TOL = 1e-5
FORMATS = [po.TT_IQ4_NL, po.TT_Q4_0, po.TT_Q8_0]
BLOCK = {po.TT_IQ4_NL: 18, po.TT_Q4_0: 18, po.TT_Q8_0: 34}


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


# the team width and pass count the library takes for a row width: at
# width 5120 Q8_0 40-lane teams of two passes, IQ4_NL 16-lane teams of five;
# else 20-lane teams where the units are a multiple of 20, then whole waves,
# 32 and 16
def geometry(cols, tt=po.TT_IQ4_NL):
    U = cols // 64
    if U == 80 and tt in (po.TT_Q8_0, po.TT_IQ4_NL):
        return (40, 2) if tt == po.TT_Q8_0 else (16, 5)
    for T, pmax in ((20, 4), (64, 2), (32, 4), (16, 4)):
        if U % T == 0 and U // T <= pmax:
            return T, U // T
    return None


def image_of(w, rows, cols, tt):
    """The documented image layout, restated on the host from the GGUF bytes:
    the 16-byte quant slots in the team's walking order (Q8_0: two per block,
    the split activation's order), then the f16 scale pairs."""
    T, P = geometry(cols, tt)
    U = T * P
    bb = BLOCK[tt]
    qs = (bb - 2) // 16
    blk = w.reshape(rows, U, 2, bb)
    u = np.arange(U)
    p, j = u // T, u % T
    q = np.zeros((rows, 2 * qs * U, 16), np.uint8)
    for e in range(2):
        for h in range(qs):
            q[:, ((2 * p + e) * qs + h) * T + j] = blk[:, :, e, 2 + 16 * h:18 + 16 * h]
    sc = np.zeros((rows, U, 4), np.uint8)
    sc[:, j * P + p, 0:2] = blk[:, :, 0, 0:2]
    sc[:, j * P + p, 2:4] = blk[:, :, 1, 0:2]
    return np.concatenate([q.reshape(rows, -1), sc.reshape(rows, -1)], axis=1)


@pytest.mark.parametrize("tt", FORMATS)
@pytest.mark.parametrize("rows,cols", [(1, 1024), (7, 2560), (5, 5120), (3, 4096), (2, 3072), (2, 6144)])
def test_image_layout(gpu, tt, rows, cols):
    w = synth.make_weight(tt, rows, cols, seed=3, tag=tt)
    img = ops.gemv_image(tt, torch.from_numpy(w).to(gpu), rows, cols).cpu().numpy()
    assert np.array_equal(img[:rows * w.shape[1]].reshape(rows, -1), image_of(w, rows, cols, tt))


@pytest.mark.parametrize("tt", [po.TT_IQ4_NL, po.TT_Q8_0])
@pytest.mark.parametrize("cols,tokens", [(1024, 1), (2560, 3), (5120, 2), (8192, 1)])
def test_split_activation_is_the_reference_quantization(gpu, tt, cols, tokens):
    x = synth.make_act(cols, tokens, seed=4)
    x[0, :32] = 0.0          # an all-zero block
    x[-1, 40] = np.float32(3e38)
    ref = ops.quantize_act(tt, torch.from_numpy(x).to(gpu)).cpu().numpy().reshape(tokens, -1)
    xa = ops.quantize_act_image(tt, torch.from_numpy(x).to(gpu)).cpu().numpy()
    T, P = geometry(cols, tt)
    U = T * P
    for t in range(tokens):
        a = xa[72 * U * t:72 * U * (t + 1)]
        blk = ref[t].reshape(U, 2, 34)
        qs = a[:64 * U].reshape(4 * U, 16)
        d = a[64 * U:].view(np.float32).reshape(U, 2)
        for u in range(U):
            p, j = u // T, u % T
            for e in range(2):
                for h in range(2):
                    assert np.array_equal(qs[((2 * p + e) * 2 + h) * T + j], blk[u, e, 2 + 16 * h:18 + 16 * h])
                assert d[j * P + p, e] == np.float32(blk[u, e, 0:2].copy().view(np.float16)[0])


@pytest.mark.parametrize("tt", FORMATS)
@pytest.mark.parametrize("rows,cols,nr", [(300, 2560, 0), (257, 1024, 0), (129, 5120, 0), (1, 2560, 0),
                                          (250, 2560, 1), (251, 2560, 2), (99, 3072, 0), (64, 8192, 2),
                                          (77, 1280, 0), (40, 6144, 1), (33, 3840, 2), (50, 2048, 0),
                                          (60, 4096, 0)])
def test_image_gemv_vs_oracle(gpu, oracle, tt, rows, cols, nr):
    w = synth.make_weight(tt, rows, cols, seed=5, tag=tt)
    x = synth.make_act(cols, 1, seed=5)
    img = ops.gemv_image(tt, torch.from_numpy(w).to(gpu), rows, cols)
    xa = ops.quantize_act_image(tt, torch.from_numpy(x).to(gpu))
    out = ops.mul_mat_vec_image(tt, img, xa, rows, cols, nr).cpu().numpy()
    want = oracle.matvec(tt, w, x)[0]
    assert rel_l2(out, want) < TOL
    # the GGUF-layout GEMV: the same integers, the same float expression per unit
    raw = ops.mul_mat(tt, torch.from_numpy(w).to(gpu), ops.quantize_act(tt, torch.from_numpy(x).to(gpu)),
                      rows, cols, 1).cpu().numpy().reshape(-1)
    assert rel_l2(out, raw) < 1e-6


@pytest.mark.parametrize("tt", FORMATS)
def test_image_gemv_integers_exact(gpu, oracle, tt):
    """Unit weight scales and integer activations of Q8_0 scale 1: every
    output is the exact sum of the row's block integers."""
    rows, cols = 96, 2560
    w = synth.make_weight(tt, rows, cols, seed=6, tag=tt).reshape(rows, -1, BLOCK[tt]).copy()
    w[:, :, 0:2] = np.array([1.0], np.float16).view(np.uint8)
    w = w.reshape(rows, -1)
    rng = np.random.default_rng(6)
    x = rng.integers(-127, 128, (1, cols)).astype(np.float32)
    x[:, ::32] = 127.0
    act = oracle.quantize_act(tt, x)
    ints = oracle.block_ints(tt, w, act, cols)[0].sum(axis=1).astype(np.float64)
    assert np.all(np.abs(ints) < 2 ** 24)
    img = ops.gemv_image(tt, torch.from_numpy(w).to(gpu), rows, cols)
    xa = ops.quantize_act_image(tt, torch.from_numpy(x).to(gpu))
    for nr in (0, 1, 2):
        out = ops.mul_mat_vec_image(tt, img, xa, rows, cols, nr).cpu().numpy().astype(np.float64)
        assert np.array_equal(out, ints)


@pytest.fixture()
def backend(gpu):
    be = ops.Backend(0)
    yield be
    be.close()


BIG = (8192, 4096)  # past the one-launch quantize + GEMV: the image path


@pytest.mark.parametrize("tt", FORMATS)
def test_backend_matvec_builds_and_reads_image(gpu, oracle, backend, tt):
    rows, cols = BIG
    w = synth.make_weight(tt, rows, cols, seed=7, tag=tt)
    x = synth.make_act(cols, 1, seed=7)
    lin = backend.load_linear(tt, rows, cols, w)
    before = backend.mem_placed()
    assert backend.prepare_linear(lin) == 0
    assert backend.mem_placed() - before >= rows * w.shape[1]  # the image
    out = torch.empty(rows, device=gpu)
    backend.matvec(out, lin, torch.from_numpy(x[0]).to(gpu))
    backend.sync()
    want = oracle.matvec(tt, w, x)[0]
    assert rel_l2(out.cpu().numpy(), want) < TOL
    # images off: the GGUF-layout launches, same result within the tolerance
    backend.set_gemv_images(False)
    out2 = torch.empty(rows, device=gpu)
    backend.matvec(out2, lin, torch.from_numpy(x[0]).to(gpu))
    backend.sync()
    assert rel_l2(out2.cpu().numpy(), want) < TOL
    backend.set_gemv_images(True)


def test_backend_matvec_pair_adjacent_images(gpu, oracle, backend):
    tt, (rows, cols) = po.TT_IQ4_NL, BIG
    wa = synth.make_weight(tt, rows, cols, seed=8, tag=1)
    wb = synth.make_weight(tt, rows, cols, seed=8, tag=2)
    x = synth.make_act(cols, 1, seed=8)
    la = backend.load_linear(tt, rows, cols, wa)
    backend.prepare_linear(la)
    lb = backend.load_linear(tt, rows, cols, wb)
    backend.prepare_linear(lb)
    out = torch.empty(2 * rows, device=gpu)
    backend.matvec_pair(out, la, lb, torch.from_numpy(x[0]).to(gpu))
    backend.sync()
    got = out.cpu().numpy()
    assert rel_l2(got[:rows], oracle.matvec(tt, wa, x)[0]) < TOL
    assert rel_l2(got[rows:], oracle.matvec(tt, wb, x)[0]) < TOL
    # the second weight alone, from inside the images
    ob = torch.empty(rows, device=gpu)
    backend.matvec(ob, lb, torch.from_numpy(x[0]).to(gpu))
    backend.sync()
    assert np.array_equal(ob.cpu().numpy(), got[rows:])


def test_backend_memo_keeps_layouts_apart(gpu, oracle, backend):
    """One x through an image matvec and a GGUF-layout matvec of the same
    activation family, in both orders, with the activation memo on."""
    rows, cols = BIG
    wi = synth.make_weight(po.TT_IQ4_NL, rows, cols, seed=9, tag=1)
    wq = synth.make_weight(po.TT_Q8_0, 256, cols, seed=9, tag=2)
    x = synth.make_act(cols, 1, seed=9)
    li = backend.load_linear(po.TT_IQ4_NL, rows, cols, wi)
    lq = backend.load_linear(po.TT_Q8_0, 256, cols, wq)
    backend.set_act_memo(True)
    xd = torch.from_numpy(x[0]).to(gpu)
    for order in ((li, lq), (lq, li), (li, li)):
        backend.step_begin(0)
        for lin in order:
            rows_l = lin.rows
            out = torch.empty(rows_l, device=gpu)
            backend.matvec(out, lin, xd)
            backend.sync()
            w = wi if lin.ttype == po.TT_IQ4_NL else wq
            assert rel_l2(out.cpu().numpy(), oracle.matvec(lin.ttype, w, x)[0]) < TOL
    backend.set_act_memo(False)


def test_backend_memo_keeps_split_layouts_apart(gpu, oracle, backend):
    """At width 5120 Q8_0 and IQ4_NL images read split activations of
    different team geometries: one x through both, in both orders, with the
    activation memo on."""
    rows, cols = 17408, 5120
    wi = synth.make_weight(po.TT_IQ4_NL, rows, cols, seed=11, tag=1)
    wq = synth.make_weight(po.TT_Q8_0, rows, cols, seed=11, tag=2)
    x = synth.make_act(cols, 1, seed=11)
    li = backend.load_linear(po.TT_IQ4_NL, rows, cols, wi)
    lq = backend.load_linear(po.TT_Q8_0, rows, cols, wq)
    backend.set_act_memo(True)
    xd = torch.from_numpy(x[0]).to(gpu)
    want = {po.TT_IQ4_NL: oracle.matvec(po.TT_IQ4_NL, wi, x)[0], po.TT_Q8_0: oracle.matvec(po.TT_Q8_0, wq, x)[0]}
    for order in ((li, lq), (lq, li), (lq, lq)):
        backend.step_begin(0)
        for lin in order:
            out = torch.empty(rows, device=gpu)
            backend.matvec(out, lin, xd)
            backend.sync()
            assert rel_l2(out.cpu().numpy(), want[lin.ttype]) < TOL
    hits, misses = backend.act_stats()
    assert (hits, misses) == (1, 5)  # only the repeat in one layout reuses the quantized x
    backend.set_act_memo(False)


def test_backend_free_linear_drops_image_of_reused_memory(gpu, oracle, backend):
    tt, (rows, cols) = po.TT_IQ4_NL, BIG
    w1 = synth.make_weight(tt, rows, cols, seed=10, tag=1)
    w2 = synth.make_weight(tt, rows, cols, seed=10, tag=2)
    x = synth.make_act(cols, 1, seed=10)
    buf = torch.from_numpy(w1.reshape(-1).copy()).to(gpu)
    xd = torch.from_numpy(x[0]).to(gpu)
    lin = backend.wrap_linear(tt, rows, cols, buf)
    out = torch.empty(rows, device=gpu)
    backend.matvec(out, lin, xd)
    backend.sync()
    assert rel_l2(out.cpu().numpy(), oracle.matvec(tt, w1, x)[0]) < TOL
    backend.free_linear(lin)
    buf.copy_(torch.from_numpy(w2.reshape(-1).copy()).to(gpu))
    lin = backend.wrap_linear(tt, rows, cols, buf)
    backend.matvec(out, lin, xd)
    backend.sync()
    assert rel_l2(out.cpu().numpy(), oracle.matvec(tt, w2, x)[0]) < TOL
