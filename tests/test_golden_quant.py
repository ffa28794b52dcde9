"""Pins the oracle's quantizers byte for byte against golden blocks produced
by the reference's own Python ports of ggml's quantizers (convert/q4k.py,
convert/q6k.py; fixtures written by tests/golden/make_quant_fixtures.py).

The ports differ from ggml's C in three documented places (see the PORT_*
bits of the oracle's quantizer); with those conventions selected the oracle
must reproduce the ports' bytes, which pins everything else: the weights of
the scale search, the candidate loop, the 6-bit scale packing, the fp16
d / dmin, the requantization and the nibble / 2-bit packing.  One Q6_K block
is a near tie of the scale search that the port (numpy pairwise sums) and
ggml (sequential sums) break differently; it is allowed to differ, and only
in that block.
"""
import pathlib

import numpy as np

import pyoracle as O

F = np.load(pathlib.Path(__file__).parent / "golden" / "quant_blocks.npz")


def diff_blocks(a, b):
    return np.nonzero((a != b).any(axis=1))[0].tolist()


def test_q4k_port_conventions_byte_exact():
    x = F["x"]
    got = O.quantize(O.TYPE_Q4_K, x, port=O.PORT_ZERO_L | O.PORT_FIXED_SPAN).reshape(len(x), -1)
    assert diff_blocks(got, F["q4k"]) == []


def test_q6k_port_conventions_byte_exact_but_one_near_tie():
    x = F["x"]
    got = O.quantize(O.TYPE_Q6_K, x, port=O.PORT_FP32_D | O.PORT_ZERO_L).reshape(len(x), -1)
    bad = diff_blocks(got, F["q6k"])
    assert bad == [22], bad
    # the near tie picks a neighbouring scale: both reconstructions are as good
    e_got = np.abs(O.dequantize(O.TYPE_Q6_K, got[22], 256) - x[22]).mean()
    e_ref = np.abs(O.dequantize(O.TYPE_Q6_K, F["q6k"][22], 256) - x[22]).mean()
    assert abs(e_got - e_ref) <= 0.02 * e_ref


def test_ggml_mode_differs_only_by_the_documented_conventions():
    # ggml semantics (the default, and what the GPU quantizer reproduces):
    # every difference from the port-convention bytes must come from the
    # span rule or the zero-scale rule, i.e. switching them on removes it
    x = F["x"]
    ggml4 = O.quantize(O.TYPE_Q4_K, x).reshape(len(x), -1)
    span_only = O.quantize(O.TYPE_Q4_K, x, port=O.PORT_FIXED_SPAN).reshape(len(x), -1)
    zero_only = O.quantize(O.TYPE_Q4_K, x, port=O.PORT_ZERO_L).reshape(len(x), -1)
    both = O.quantize(O.TYPE_Q4_K, x, port=O.PORT_FIXED_SPAN | O.PORT_ZERO_L).reshape(len(x), -1)
    touched = set(diff_blocks(ggml4, span_only)) | set(diff_blocks(ggml4, zero_only))
    assert set(diff_blocks(ggml4, both)) <= touched
    # the zero-scale rule only acts on blocks with a zero 6-bit scale; their
    # dequantized values are identical either way
    for b in diff_blocks(ggml4, zero_only):
        assert np.array_equal(O.dequantize(O.TYPE_Q4_K, ggml4[b], 256),
                              O.dequantize(O.TYPE_Q4_K, zero_only[b], 256))
