"""GPU: the Exec mirror's activation-quantization memo (backend_cuda.zig:3425-3448,
:3914-3944), the decode-step hints (backend.zig:470-491) and a decode step
captured in a HIP graph by the caller and replayed.

For widths up to 4096 the mirror quantizes inside the GEMV (one fused
launch); with the memo on, that launch also leaves the quantized rows in the
scratch, so a memo hit then runs the plain GEMV on them.  The two kernels fold
the block terms in different orders, so results are compared to 1e-6 relative
L2 where a hit replaces a fused launch, and bit for bit where the same kernel
runs."""
import numpy as np
import pytest
import torch

import pyoracle as po
from qwen35_amd import ops, synth

pytestmark = pytest.mark.gpu
TOL = 1e-5
COLS = 2560


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


@pytest.fixture(scope="module")
def weights():
    up = synth.make_weight(po.TT_Q4_K, 9728, COLS, seed=31, tag=po.TT_Q4_K)
    gate = synth.make_weight(po.TT_Q4_K, 9728, COLS, seed=32, tag=po.TT_Q4_K)
    q6 = synth.make_weight(po.TT_Q6_K, 2560, COLS, seed=33, tag=po.TT_Q6_K)
    down = synth.make_weight(po.TT_Q6_K, 2560, 9728, seed=34, tag=po.TT_Q6_K)
    return up, gate, q6, down


def test_memo_hits_same_family_and_matches(gpu, oracle, weights):
    up, _, q6, _ = weights
    be = ops.Backend(0)
    try:
        lu = be.load_linear(po.TT_Q4_K, 9728, COLS, up)
        l6 = be.load_linear(po.TT_Q6_K, 2560, COLS, q6)
        x = synth.make_act(COLS, 1, seed=35)
        xd = torch.from_numpy(x[0]).to(gpu)
        want_u, want_6 = oracle.matvec(po.TT_Q4_K, up, x)[0], oracle.matvec(po.TT_Q6_K, q6, x)[0]
        # memo off: every matvec quantizes, nothing is counted
        ou0, o60 = torch.empty(9728, device=gpu), torch.empty(2560, device=gpu)
        be.matvec(ou0, lu, xd)
        be.matvec(o60, l6, xd)
        be.sync()
        assert be.act_stats() == (0, 0)
        be.set_act_memo(True)
        be.step_begin(0)
        ou, o6 = torch.empty(9728, device=gpu), torch.empty(2560, device=gpu)
        be.matvec(ou, lu, xd)   # miss: quantized to Q8_K
        be.matvec(o6, l6, xd)   # Q6_K takes the same Q8_K rows: hit
        be.sync()
        assert be.act_stats() == (1, 1)
        # the memo only skips work: the miss ran the same fused launch as the
        # memo-off call; the hit ran the plain GEMV on the same quantized rows
        assert torch.equal(ou, ou0)
        assert rel_l2(o6.cpu().numpy(), o60.cpu().numpy()) < 1e-6
        assert rel_l2(ou.cpu().numpy(), want_u) < TOL
        assert rel_l2(o6.cpu().numpy(), want_6) < TOL
        # another pointer, or another width, or a new step: miss
        x2 = xd.clone()
        be.matvec(o6, l6, x2)
        be.step_begin(1)
        be.matvec(o6, l6, x2)
        be.sync()
        assert be.act_stats() == (1, 3)
        assert torch.equal(o6, o60)
    finally:
        be.close()


def test_memo_invalidate_after_write(gpu, oracle, weights):
    _, _, q6, _ = weights
    be = ops.Backend(0)
    try:
        l6 = be.load_linear(po.TT_Q6_K, 2560, COLS, q6)
        x = synth.make_act(COLS, 1, seed=36)
        xd = torch.from_numpy(x[0]).to(gpu)
        be.set_act_memo(True)
        o_a, o_b, o_c = (torch.empty(2560, device=gpu) for _ in range(3))
        be.matvec(o_a, l6, xd)
        xd.mul_(-0.5)            # a write into x the memo cannot see ...
        be.matvec(o_b, l6, xd)   # ... so it reuses the old rows (the documented contract)
        be.act_invalidate()
        be.matvec(o_c, l6, xd)
        be.sync()
        assert rel_l2(o_b.cpu().numpy(), o_a.cpu().numpy()) < 1e-6
        x_new = (x[0] * np.float32(-0.5))[None, :]
        assert rel_l2(o_c.cpu().numpy(), oracle.matvec(po.TT_Q6_K, q6, x_new)[0]) < TOL
        assert be.act_stats() == (1, 2)
        # set_act_memo(False) stops reuse
        be.set_act_memo(False)
        xd.mul_(-2.0)
        be.matvec(o_b, l6, xd)
        be.sync()
        assert rel_l2(o_b.cpu().numpy(), oracle.matvec(po.TT_Q6_K, q6, x)[0]) < TOL
    finally:
        be.close()


def test_memo_non_adjacent_pair_quantizes_once(gpu, oracle, weights):
    up, gate, _, _ = weights
    be = ops.Backend(0)
    try:
        lu = be.load_linear(po.TT_Q4_K, 9728, COLS, up)
        gd = torch.from_numpy(gate).to(gpu)
        lg = be.wrap_linear(po.TT_Q4_K, 9728, COLS, gd)   # not adjacent: two GEMVs
        x = synth.make_act(COLS, 1, seed=37)
        xd = torch.from_numpy(x[0]).to(gpu)
        be.set_act_memo(True)
        out = torch.empty(2 * 9728, device=gpu)
        be.matvec_pair(out, lu, lg, xd)
        be.sync()
        assert be.act_stats() == (1, 1)
        want = np.concatenate([oracle.matvec(po.TT_Q4_K, up, x)[0], oracle.matvec(po.TT_Q4_K, gate, x)[0]])
        assert rel_l2(out.cpu().numpy(), want) < TOL
    finally:
        be.close()


def test_decode_step_in_hip_graph(gpu, oracle, weights):
    """gate/up pair + down captured once by the caller, replayed with new
    activations written between replays; every replay checked."""
    up, gate, _, down = weights
    be = ops.Backend(0)
    try:
        lg = be.load_linear(po.TT_Q4_K, 9728, COLS, gate)
        lu = be.load_linear(po.TT_Q4_K, 9728, COLS, up)   # adjacent: one launch
        ld = be.load_linear(po.TT_Q6_K, 2560, 9728, down)
        be.set_act_memo(True)
        xd = torch.zeros(COLS, device=gpu)
        hd = torch.zeros(9728, device=gpu)
        gu = torch.empty(2 * 9728, device=gpu)
        y = torch.empty(2560, device=gpu)

        def step(pos):
            be.step_begin(pos)
            be.matvec_pair(gu, lg, lu, xd)
            be.matvec(y, ld, hd)
            be.step_end()

        step(0)                      # warm-up: scratch allocated outside the capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            be.set_stream(torch.cuda.current_stream())
            step(0)
        be.set_stream(torch.cuda.current_stream())
        torch.cuda.synchronize()
        # a prefill after the capture grows the activation scratch and the
        # split-K workspace past what the graph was captured with; the buffers
        # the graph names must stay valid for its replays
        placed = be.mem_placed()
        hk = synth.make_act(9728, 64, seed=500)
        yk = torch.empty((64, 2560), device=gpu)
        be.matvec_batch_k(yk, ld, torch.from_numpy(hk).to(gpu), 64)
        torch.cuda.synchronize()
        assert be.mem_placed() > placed
        assert rel_l2(yk.cpu().numpy(), oracle.matvec(po.TT_Q6_K, down, hk)) < TOL
        for rep in range(4):
            x = synth.make_act(COLS, 1, seed=300 + rep)
            h = synth.make_act(9728, 1, seed=400 + rep)
            xd.copy_(torch.from_numpy(x[0]))
            hd.copy_(torch.from_numpy(h[0]))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            want_gu = np.concatenate([oracle.matvec(po.TT_Q4_K, gate, x)[0],
                                      oracle.matvec(po.TT_Q4_K, up, x)[0]])
            assert rel_l2(gu.cpu().numpy(), want_gu) < TOL, rep
            assert rel_l2(y.cpu().numpy(), oracle.matvec(po.TT_Q6_K, down, h)[0]) < TOL, rep
            # eager step on the same buffers between replays gives the same numbers
            gu_r, y_r = gu.clone(), y.clone()
            step(rep + 1)
            torch.cuda.synchronize()
            assert torch.equal(gu, gu_r) and torch.equal(y, y_r), rep
        del g
    finally:
        torch.cuda.synchronize()
        be.close()
