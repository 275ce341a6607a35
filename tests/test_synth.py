"""The synthetic-input generator is deterministic and follows the configs' block rules."""
import numpy as np

from qwen35_amd import synth


def test_splitmix64_known_values():
    # SplitMix64, seed 0: published first outputs
    z = synth.splitmix64(0, 3)
    assert [int(v) for v in z] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_deterministic_and_seeded():
    a = synth.make_weight(synth.TT_Q4_K, 16, 512, seed=0)
    b = synth.make_weight(synth.TT_Q4_K, 16, 512, seed=0)
    c = synth.make_weight(synth.TT_Q4_K, 16, 512, seed=1)
    assert synth.sha256(a) == synth.sha256(b) != synth.sha256(c)


def test_block_rules():
    w = synth.make_weight(synth.TT_Q8_0, 64, 1024).reshape(-1, 34)
    q = w[:, 2:].view(np.int8)
    assert q.min() >= -127 and q.max() <= 127
    d = w[:, 0:2].copy().view(np.float16).astype(np.float32)
    assert np.all(d >= 0) and 1e-4 < float(np.median(d)) < 2e-4
    w6 = synth.make_weight(synth.TT_Q6_K, 32, 512).reshape(-1, 210)
    sc = w6[:, 192:208].view(np.int8)
    assert sc.min() >= -64 and sc.max() <= 63
    x = synth.make_act(4096, 2)
    assert abs(float(x.mean())) < 0.05 and abs(float(x.std()) - 1) < 0.05


def test_ragged_lengths_and_offsets():
    lens = synth.ragged_lengths(8, 16, 256, seed=0)
    assert lens.min() >= 16 and lens.max() <= 256
    off = synth.offsets_from_lengths(lens)
    assert off[0] == 0 and off[-1] == lens.sum() and np.all(np.diff(off) == lens)
