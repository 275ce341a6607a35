"""GPU: GGUF blocks -> f32 (q35_launch_dequantize / _row, Exec.dequantRow),
bit-exact against the oracle's restatement of src/quant_dequant.zig, which the
reference's own udtest fixtures pin (tests/test_oracle_pins.py)."""
import numpy as np
import pytest
import torch

import pyoracle as po
import qwen35_amd
from qwen35_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu
TYPES = po.ALL_TYPES


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def with_edge_scales(tt, w):
    """Overwrite some block scales with f16 edge values: subnormal, negative,
    zero, -0 and the largest finite."""
    be, bb = po.GEOM[tt]
    blk = w.reshape(-1, bb).copy()
    edge = np.array([0x0001, 0x03FF, 0x8400, 0x0000, 0x8000, 0x7BFF, 0xFBFF], np.uint16).view(np.uint8)
    n = min(len(blk), 7)
    off = {po.TT_Q6_K: 208, po.TT_Q3_K: 108, po.TT_Q2_K: 80}.get(tt, 0)
    blk[:n, off:off + 2] = edge.reshape(-1, 2)[:n]
    dmin = {po.TT_Q4_K: 2, po.TT_Q5_K: 2, po.TT_Q2_K: 82, po.TT_Q4_1: 2}.get(tt)
    if dmin is not None:
        blk[:n, dmin:dmin + 2] = edge.reshape(-1, 2)[::-1][:n]
    return blk.reshape(w.shape)


@pytest.mark.parametrize("tt", TYPES)
def test_dequantize_rows_bit_exact(gpu, oracle, tt):
    rows, cols = 7, 2560 if tt not in (po.TT_Q6_K, po.TT_Q3_K) else 2304
    w = with_edge_scales(tt, synth.make_weight(tt, rows, cols, seed=4, tag=tt))
    wd = to_dev(w, gpu)
    for r in range(rows):
        got = ops.dequantize_row(tt, wd[r], cols).cpu().numpy()
        want = oracle.dequant_row(tt, w[r], cols)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), r


@pytest.mark.parametrize("tt", TYPES)
def test_dequantize_blocks_whole_tensor(gpu, oracle, tt):
    rows, cols = 33, 1024
    w = synth.make_weight(tt, rows, cols, seed=5, tag=tt)
    nblocks = rows * cols // po.GEOM[tt][0]
    got = ops.dequantize(tt, to_dev(w, gpu), nblocks).cpu().numpy().reshape(rows, cols)
    want = np.stack([oracle.dequant_row(tt, w[r], cols) for r in range(rows)])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_backend_dequant_row(gpu, oracle):
    tt, rows, cols = po.TT_Q4_K, 12, 2560
    w = synth.make_weight(tt, rows, cols, seed=6, tag=tt)
    be = ops.Backend(0)
    try:
        lin = be.load_linear(tt, rows, cols, w)
        out = torch.empty(cols, device=gpu)
        for r in (0, 5, rows - 1):
            be.dequant_row(out, lin, r)
            be.sync()
            assert np.array_equal(out.cpu().numpy(), oracle.dequant_row(tt, w[r], cols))
        with pytest.raises(qwen35_amd.QhipError):
            be.dequant_row(out, lin, rows)  # row out of range
    finally:
        be.close()


def test_dequantize_rejects_bad_arguments(gpu):
    L = _lib.load()
    buf = torch.zeros(1024, dtype=torch.uint8, device=gpu)
    out = torch.empty(256, device=gpu)
    assert L.qhip_launch_dequantize_row(po.TT_Q4_K, buf.data_ptr(), out.data_ptr(), 100, None) != 0
    assert L.qhip_launch_dequantize_row(99, buf.data_ptr(), out.data_ptr(), 256, None) != 0
    assert L.qhip_launch_dequantize(po.TT_Q8_0, buf.data_ptr(), out.data_ptr(), -1, None) != 0
    assert L.qhip_launch_dequantize(po.TT_Q8_0, buf.data_ptr(), out.data_ptr(), 0, None) == 0
