"""Seeded input generator: SplitMix64 against its published test vectors,
and the Box-Muller normals' moments."""
import numpy as np

from ullm_amd import synth


def test_splitmix64_reference_outputs():
    # Vigna's splitmix64.c: the first outputs from state 0 and from 1234567
    assert int(synth.splitmix64(0, 1)[0]) == 0xE220A8397B1DCDAF
    assert [int(x) for x in synth.splitmix64(1234567, 5)] == [
        6457827717110365317, 3203168211198807973, 9817491932198370423,
        4593380528125082431, 16408922859458223821]


def test_normals_are_standard_and_deterministic():
    z = synth.normal(42, 200001)
    assert z.dtype == np.float32 and z.shape == (200001,)
    assert abs(float(z.mean())) < 0.01 and abs(float(z.std()) - 1) < 0.01
    np.testing.assert_array_equal(z, synth.normal(42, 200001))
    assert not np.array_equal(synth.normal(substream := synth.substream(1, 1), 10),
                              synth.normal(synth.substream(1, 2), 10))


def test_ragged_lengths_in_range():
    ls = synth.ragged_lengths(5, 64, 4096, 32768)
    assert min(ls) >= 4096 and max(ls) <= 32768 and len(set(ls)) > 50
