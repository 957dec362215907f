"""The seeded generator: SplitMix64 known answers and block-format invariants."""
import numpy as np

from moe_rocm import synth as S
from moe_rocm import workloads as W


def test_splitmix64_known_answers():
    # Published SplitMix64 outputs for seed 0 (Vigna's splitmix64.c reference).
    d = S.draws(0, 0, 3)
    assert [int(v) for v in d] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_counter_form_is_stream_suffix():
    a = S.draws(12345, 0, 100)
    b = S.draws(12345, 37, 63)
    assert np.array_equal(a[37:], b)


def test_mxfp4_blocks_format():
    blk = S.mxfp4_blocks(S.stream_seed(1, 2, 3, 4), 20000).reshape(-1, 17)
    assert blk[:, 0].min() == 119 and blk[:, 0].max() == 127
    nib = np.concatenate([blk[:, 1:] & 15, blk[:, 1:] >> 4]).reshape(-1)
    counts = np.bincount(nib, minlength=16)
    assert counts.min() > 0.9 * counts.mean()
    part = S.mxfp4_blocks(S.stream_seed(1, 2, 3, 4), 100, first_block=500)
    assert np.array_equal(part, blk[500:600].reshape(-1))


def test_q4k_blocks_format():
    blk = S.q4k_blocks(S.stream_seed(5, 6, 7, 8), 4000).reshape(-1, 144)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float64).ravel()
    dm = blk[:, 2:4].copy().view(np.float16).astype(np.float64).ravel()
    assert np.all(d >= 0) and np.all(dm >= 0)
    # |N(0, s)| has mean s*sqrt(2/pi)
    assert abs(d.mean() / (0.01 * np.sqrt(2 / np.pi)) - 1) < 0.05
    assert abs(dm.mean() / (0.005 * np.sqrt(2 / np.pi)) - 1) < 0.05
    part = S.q4k_blocks(S.stream_seed(5, 6, 7, 8), 10, first_block=77)
    assert np.array_equal(part, blk[77:87].reshape(-1))


def test_normal_moments():
    z = S.normal(S.stream_seed(9), 200000, 1.0).astype(np.float64)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01


def test_config_shapes_and_bytes():
    c2 = W.config_layers(2)
    assert len(c2) == 24 and c2[0].hidden == 2880 and c2[0].top_k == 4
    # algorithmic bytes per C1 layer-token (MXFP4 weights + biases + router + x/y)
    assert c2[0].weight_bytes_per_token() == 53_406_720 + 128
    c3 = W.config_layers(3)
    # C3 per layer-token: 8 experts x 3 x 884,736 B + router 128 x 2048 x 4 B + x/y 2 x 8,192 B
    assert c3[0].weight_bytes_per_token() == 8 * 3 * 884_736 + 1_048_576 + 16_384 == 22_298_624
    assert sum(s.weight_bytes_per_token() for s in c3) == 48 * 22_298_624 == 1_070_333_952
    c4 = W.config_layers(4)
    assert len(c4) == 48 and all(256 <= s.n_experts <= 512 for s in c4)
    assert len({s.n_experts for s in c4}) > 10
    lp = W.zipf_log_p(W.config_layers(5)[0])
    assert abs(np.exp(lp).sum() - 1) < 1e-12 and len(set(np.round(lp, 9))) == 32
