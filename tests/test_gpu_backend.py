"""GPU: the Exec-slot mirror (matvec / matvecPair / matvecBatchK), the ragged
packer + ragged launch, and the full-size BASELINE configurations checked on
sampled rows (a size-independent property: any row of the full launch equals
the oracle's row)."""
import numpy as np
import pytest
import torch

import pyoracle as po
from qwen35_amd import ops, synth

pytestmark = pytest.mark.gpu
TOL = 1e-5


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


@pytest.fixture(scope="module")
def backend(gpu):
    be = ops.Backend(0)
    yield be
    be.close()


@pytest.mark.parametrize("tt,rows,cols", [(po.TT_Q8_0, 256, 1024), (po.TT_Q4_K, 128, 2560),
                                          (po.TT_Q6_K, 64, 9728), (po.TT_IQ4_NL, 96, 2560),
                                          (po.TT_Q5_K, 128, 2560), (po.TT_Q3_K, 80, 2304),
                                          (po.TT_Q2_K, 96, 2560), (po.TT_IQ4_XS, 112, 2560),
                                          (po.TT_Q4_0, 96, 2560), (po.TT_Q4_1, 96, 2560),
                                          (po.TT_IQ3_XXS, 96, 2560), (po.TT_IQ3_S, 96, 2560)])
def test_backend_matvec(gpu, oracle, backend, tt, rows, cols):
    w = synth.make_weight(tt, rows, cols, seed=21, tag=tt)
    x = synth.make_act(cols, 1, seed=21)
    lin = backend.load_linear(tt, rows, cols, w)
    out = torch.empty(rows, device=gpu)
    backend.matvec(out, lin, torch.from_numpy(x[0]).to(gpu))
    backend.sync()
    assert rel_l2(out.cpu().numpy(), oracle.matvec(tt, w, x)[0]) < TOL


def test_backend_matvec_pair_adjacent_and_not(gpu, oracle, backend):
    tt, rows, cols = po.TT_Q4_K, 96, 2560
    a = synth.make_weight(tt, rows, cols, seed=1, tag=1)
    b = synth.make_weight(tt, rows, cols, seed=2, tag=2)
    x = synth.make_act(cols, 1, seed=3)
    want = np.concatenate([oracle.matvec(tt, a, x)[0], oracle.matvec(tt, b, x)[0]])
    la = backend.load_linear(tt, rows, cols, a)
    lb = backend.load_linear(tt, rows, cols, b)  # arena: adjacent to la
    assert lb.dev == la.dev + rows * la.row_bytes
    xd = torch.from_numpy(x[0]).to(gpu)
    out = torch.empty(2 * rows, device=gpu)
    backend.matvec_pair(out, la, lb, xd)
    backend.sync()
    assert rel_l2(out.cpu().numpy(), want) < TOL
    # not adjacent: a separate allocation for b
    bd = torch.from_numpy(b).to(gpu)
    lb2 = backend.wrap_linear(tt, rows, cols, bd)
    out2 = torch.empty(2 * rows, device=gpu)
    backend.matvec_pair(out2, la, lb2, xd)
    backend.sync()
    assert rel_l2(out2.cpu().numpy(), want) < TOL


@pytest.mark.parametrize("k", [1, 7, 16])
@pytest.mark.parametrize("tt", [po.TT_Q6_K, po.TT_Q5_K, po.TT_IQ4_XS, po.TT_IQ3_XXS])
def test_backend_batch_k(gpu, oracle, backend, k, tt):
    rows, cols = 80, 2560
    w = synth.make_weight(tt, rows, cols, seed=5, tag=tt)
    x = synth.make_act(cols, k, seed=5)
    lin = backend.load_linear(tt, rows, cols, w)
    out = torch.empty((k, rows), device=gpu)
    backend.matvec_batch_k(out, lin, torch.from_numpy(x).to(gpu), k)
    backend.sync()
    assert rel_l2(out.cpu().numpy(), oracle.matvec(tt, w, x)) < TOL


@pytest.mark.parametrize("tt", [po.TT_Q8_0, po.TT_Q4_K])
def test_ragged_pack_and_launch(gpu, oracle, tt):
    rows, cols = 192, 1024
    lens = [int(v) for v in synth.ragged_lengths(8, 16, 64, seed=tt)] + [0, 3]
    w = synth.make_weight(tt, rows, cols, seed=7, tag=tt)
    seqs = [synth.make_act(cols, n, seed=100 + i) if n else np.zeros((0, cols), np.float32)
            for i, n in enumerate(lens)]
    dseqs = [torch.from_numpy(s).to(gpu) if len(s) else torch.empty((0, cols), device=gpu) for s in seqs]
    xq, off_d, total = ops.quantize_ragged(tt, dseqs, cols)
    assert total == sum(lens)
    packed = np.concatenate(seqs)
    assert np.array_equal(xq[:total].cpu().numpy(), oracle.quantize_act(tt, packed))
    wd = torch.from_numpy(w).to(gpu)
    out = ops.mul_mat_ragged(tt, wd, xq, off_d, len(lens), total, rows, cols).cpu().numpy()
    assert rel_l2(out, oracle.matvec(tt, w, packed)) < TOL


# ---- full-size configurations, sampled rows ---------------------------------------

FULL = [("cfg1-q8_0-attn_qkv", po.TT_Q8_0, 6144, 1024),
        ("cfg2a-q4_k-ffn_up", po.TT_Q4_K, 9728, 2560),
        ("cfg2b-q6_k-ffn_down", po.TT_Q6_K, 2560, 9728),
        ("cfg3-iq4_nl-lm_head", po.TT_IQ4_NL, 248320, 2560),
        ("cfg5-q4_k-ffn_up", po.TT_Q4_K, 17408, 5120),
        ("cfg5-q6_k-ffn_down", po.TT_Q6_K, 5120, 17408)]


@pytest.mark.parametrize("name,tt,rows,cols", FULL, ids=[f[0] for f in FULL])
def test_full_size_sampled_rows(gpu, oracle, name, tt, rows, cols):
    w = synth.make_weight(tt, rows, cols, seed=0, tag=tt)
    x = synth.make_act(cols, 1, seed=0)
    wd = torch.from_numpy(w).to(gpu)
    xq = ops.quantize_act(tt, torch.from_numpy(x).to(gpu))
    out = ops.mul_mat(tt, wd, xq, rows, cols, 1).cpu().numpy()[0]
    rng = np.random.default_rng(rows)
    idx = np.unique(np.concatenate([[0, rows - 1], rng.integers(0, rows, 512)]))
    want = oracle.matvec(tt, w[idx], x)[0]
    assert rel_l2(out[idx], want) < TOL
    assert np.all(np.isfinite(out))
    sel = torch.from_numpy(idx[:64]).to(gpu)
    ints = ops.block_ints(tt, wd[sel].contiguous(), xq, len(sel), cols, 1).cpu().numpy()
    assert np.array_equal(ints, oracle.block_ints(tt, w[idx[:64]], oracle.quantize_act(tt, x), cols))
