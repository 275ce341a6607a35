"""GPU: the Exec mirror's introspection and profiling entries -- describe()
(src/backend.zig:494-495) and the device-timed slot table behind the
profiling slots (src/backend.zig:500-514; the reference's per-type device
table, src/backend_cuda.zig:6647) -- through the C ABI.

The table must count every timed call once under its (slot, type, rows,
cols, tokens) key, sum exactly the algorithmic bytes and int8 ops of those
calls, hold a positive device time for each, leave the products' results
unchanged, and skip (but count) calls made under a graph capture."""
import numpy as np
import pytest
import torch

import pyoracle as po
from qwen35_amd import ops, synth

pytestmark = pytest.mark.gpu
TOL = 1e-5
SLOT = {"matvec": 0, "pair": 1, "batch_k": 2, "dequant_row": 3}


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


def test_prof_table_counts_bytes_and_results(gpu, oracle):
    tt4, tt6 = po.TT_Q4_K, po.TT_Q6_K
    up = synth.make_weight(tt4, 1024, 2560, seed=81, tag=tt4)
    gate = synth.make_weight(tt4, 1024, 2560, seed=82, tag=tt4)
    down = synth.make_weight(tt6, 2560, 4096, seed=83, tag=tt6)
    be = ops.Backend(0)
    try:
        lu = be.load_linear(tt4, 1024, 2560, up)
        lg = be.load_linear(tt4, 1024, 2560, gate)  # adjacent: one launch for the pair
        ld = be.load_linear(tt6, 2560, 4096, down)
        assert "profiling off" in be.describe()
        be.set_profiling(True)
        x = synth.make_act(2560, 1, seed=84)
        h = synth.make_act(4096, 16, seed=85)
        xd, hd = torch.from_numpy(x[0]).to(gpu), torch.from_numpy(h).to(gpu)
        o1 = torch.empty(1024, device=gpu)
        o2 = torch.empty(2048, device=gpu)
        o3 = torch.empty((16, 2560), device=gpu)
        row = torch.empty(2560, device=gpu)
        for _ in range(3):
            be.matvec(o1, lu, xd)
        for _ in range(2):
            be.matvec_pair(o2, lu, lg, xd)
            be.matvec_batch_k(o3, ld, hd, 16)
        be.dequant_row(row, lu, 5)
        be.sync()
        # results as without profiling
        assert rel_l2(o1.cpu().numpy(), oracle.matvec(tt4, up, x)[0]) < TOL
        want2 = np.concatenate([oracle.matvec(tt4, up, x)[0], oracle.matvec(tt4, gate, x)[0]])
        assert rel_l2(o2.cpu().numpy(), want2) < TOL
        assert rel_l2(o3.cpu().numpy(), oracle.matvec(tt6, down, h)) < TOL
        assert np.array_equal(row.cpu().numpy(), oracle.dequant_row(tt4, up[5], 2560))

        ent = {(e["slot"], e["ttype"], e["rows"], e["cols"], e["tokens"]): e for e in be.prof_entries()}
        rb4, rb6 = 2560 // 256 * 144, 4096 // 256 * 210
        want = {  # key: (calls, bytes per call, ops per call)
            (SLOT["matvec"], tt4, 1024, 2560, 1): (3, 1024 * rb4 + 4 * (2560 + 1024), 2 * 1024 * 2560),
            (SLOT["pair"], tt4, 2048, 2560, 1): (2, 2048 * rb4 + 4 * (2560 + 2048), 2 * 2048 * 2560),
            (SLOT["batch_k"], tt6, 2560, 4096, 16): (2, 2560 * rb6 + 4 * (4096 + 2560) * 16,
                                                    2 * 2560 * 4096 * 16),
            (SLOT["dequant_row"], tt4, 1, 2560, 1): (1, rb4 + 4 * 2560, 0),
        }
        assert set(ent) == set(want)
        for k, (calls, nbytes, ops_) in want.items():
            e = ent[k]
            assert e["calls"] == calls, k
            assert e["bytes"] == calls * nbytes, k
            assert e["ops"] == calls * ops_, k
            assert 0.5 < e["device_us"] / calls < 1e4, (k, e["device_us"])
        # largest total first
        totals = [e["device_us"] for e in be.prof_entries()]
        assert totals == sorted(totals, reverse=True)
        text = be.prof_report()
        lines = text.strip().splitlines()
        assert lines[0].startswith("HIP-PROF ") and "calls=8" in lines[0]
        assert len(lines) == 1 + len(want)
        assert any("matvecBatchK" in l and "Q6_K" in l and "k=16" in l for l in lines)
        d = be.describe()
        assert "gfx950" in d and "profiling on" in d and "weights" in d
        # a reset empties the table; profiling off records nothing
        be.prof_reset()
        assert be.prof_entries() == []
        be.set_profiling(False)
        be.matvec(o1, lu, xd)
        be.sync()
        assert be.prof_entries() == []
    finally:
        be.close()


def test_prof_skips_captured_calls(gpu, oracle):
    tt = po.TT_Q4_K
    w = synth.make_weight(tt, 1024, 2560, seed=86, tag=tt)
    be = ops.Backend(0)
    try:
        lin = be.load_linear(tt, 1024, 2560, w)
        be.set_profiling(True)
        xd = torch.zeros(2560, device=gpu)
        out = torch.empty(1024, device=gpu)
        be.matvec(out, lin, xd)  # eager: timed, scratch allocated outside the capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            be.set_stream(torch.cuda.current_stream())
            be.matvec(out, lin, xd)
        be.set_stream(torch.cuda.current_stream())
        assert be.prof_untimed() == 1
        x = synth.make_act(2560, 1, seed=87)
        xd.copy_(torch.from_numpy(x[0]))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert rel_l2(out.cpu().numpy(), oracle.matvec(tt, w, x)[0]) < TOL
        ent = be.prof_entries()
        assert len(ent) == 1 and ent[0]["calls"] == 1
        del g
    finally:
        torch.cuda.synchronize()
        be.close()
