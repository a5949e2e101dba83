"""The fixture input generator (oracle/inputs.py) against published values and
library conversions, so fixtures regenerate identically anywhere."""
import numpy as np
import torch

from oracle import inputs


def test_splitmix64_known_answers():
    # splitmix64 with state 0: the first outputs published with the algorithm
    # (Vigna's reference implementation, seed 0).
    state = np.array([0], dtype=np.uint64)
    outs = []
    with np.errstate(over="ignore"):
        for _ in range(3):
            outs.append(int(inputs.splitmix64(state)[0]))
            state = state + inputs._GOLDEN
    assert outs == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_bf16_rounding_matches_torch():
    x = np.concatenate([inputs.normal_f32(1, 100000),
                        np.array([0.0, -0.0, 1.0, np.inf, -np.inf, 3.0e38, 1e-40, 65504.0,
                                  1.00390625, 1.01171875], dtype=np.float32)])
    ours = inputs.f32_to_bf16_bits(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)


def test_normal_statistics_and_stability():
    z = inputs.normal_f32(42, 1 << 18)
    assert abs(float(z.mean())) < 0.01 and abs(float(z.std()) - 1.0) < 0.01
    assert np.array_equal(z[100:200], inputs.normal_f32(42, 100, offset=100))
    assert not np.array_equal(z[:100], inputs.normal_f32(43, 100))


def test_id_generators():
    ids = inputs.distinct_ids(7, 1024, 4096)
    assert len(np.unique(ids)) == 1024 and ids.min() >= 0 and ids.max() < 4096
    assert np.array_equal(ids, inputs.distinct_ids(7, 1024, 4096))
    for run in (1, 8, 64, 1024):
        r = inputs.run_ids(3, 1024, 4096, run)
        assert len(np.unique(r)) == 1024
        runs = r.reshape(-1, run)
        assert np.all(np.diff(runs, axis=1) == 1)
        assert np.all(runs[:, 0] % run == 0)
