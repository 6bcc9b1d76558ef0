"""The oracle's block decoding against the reference's golden vectors.

tests/golden/quantization_q.json holds the reference's own fixture cases
(gguf-decoded floats for real-quantizer and random-byte blocks); the bar is
bit-exact, tighter than the reference's 1e-4 (DequantizerParityTests.cs:28).
"""
import numpy as np
import pytest

from helpers import quant_fixtures
from oracle import oracle

FIX = quant_fixtures()


@pytest.mark.parametrize("name", ["Q4_0", "Q5_1", "Q8_0"])
@pytest.mark.parametrize("kind", ["quantized", "synthetic"])
def test_dequant_matches_fixture_bit_exact(name, kind):
    t, entry = FIX[name]
    raw, expected = entry[kind]
    got = oracle.dequantize(t, raw, expected.size)
    assert np.array_equal(got.view(np.uint32), expected.view(np.uint32))


def test_dequant_closed_forms():
    # Q8_0: d = 0.5, q = -3 -> -1.5 ; Q4_0: d = 2, nibble 0 -> -16 ; Q5_1: d = 1, m = 0.25, q = 31 -> 31.25
    q8 = np.zeros(34, np.uint8)
    q8[0:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    q8[2] = np.uint8(np.int8(-3).view(np.uint8))
    assert oracle.dequantize(8, q8, 32)[0] == -1.5
    q4 = np.zeros(18, np.uint8)
    q4[0:2] = np.frombuffer(np.float16(2.0).tobytes(), np.uint8)
    v = oracle.dequantize(2, q4, 32)
    assert v[0] == -16.0 and v[16] == -16.0
    q5 = np.zeros(24, np.uint8)
    q5[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    q5[2:4] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
    q5[4:8] = np.frombuffer(np.uint32(1 << 17).tobytes(), np.uint8)  # fifth bit of element 17
    q5[8 + 1] = 0xF0  # element 17's high nibble = 15
    v = oracle.dequantize(7, q5, 32)
    assert v[17] == 31.25 and v[0] == 0.25


def test_dequant_rejects_partial_blocks():
    with pytest.raises(ValueError):
        oracle.dequantize(8, np.zeros(34, np.uint8), 31)
