"""Host side of the residual codec in libt5hip.so (no GPU needed): the decode table and the
exact encode thresholds the kernels use, against the CPU oracle's restatement of
src/packops.rs (make_q4_dequant_table :14-25; compand :136-142 + quantize(4) :156-162)."""
import numpy as np

from oracle import oracle as orc
from witchcraft_amd import codec


def test_table_is_the_reference_table():
    assert np.array_equal(codec.make_q4_dequant_table(), orc.q4_dequant_table())


def test_thresholds_reproduce_the_quantizer_on_every_f32():
    """code(x) = #{t_j <= x} equals compand().quantize(4) for all 2^32 bit patterns (NaN -> 0)."""
    t = codec.q4_compand_thresholds()
    assert np.all(np.diff(t.astype(np.float64)) > 0)
    bad, first = orc.ladder_mismatches(t)
    assert bad == 0, f"{bad} mismatches, first at bits {first:#010x}"


def test_thresholds_are_tight():
    """Each threshold is the least f32 with its code: one ulp below it the code drops."""
    t = codec.q4_compand_thresholds()
    for j, x in enumerate(t, start=1):
        below = np.nextafter(np.float32(x), np.float32(-np.inf))
        assert orc.compand_q4(float(x)) >= j and orc.compand_q4(float(below)) < j
