"""The oracle's FP6 e3m2 chunk form of INT4 codes (the operand of pk_gemm
format 9), pinned on the CPU:

* e3m2 decoding against the OCP Microscaling Formats (MX) v1.0 figures for
  E3M2: largest normal 28.0, smallest normal 0.25, smallest subnormal 0.0625,
  no infinities or NaN (every one of the 64 codes finite), and the 32
  non-negative codes strictly increasing;
* every integer code -8..8 encodes exactly and decodes back;
* the chunk layout, unpacked bit by bit (16 fields of 6 bits from the first 12
  bytes, little-endian), gives back the codes, with 4 zero bytes per chunk.

The device encoders (the LayerNorm producer, pk_unpack_int4_fp6) are compared
with this form bit for bit in tests/test_gpu_fp6.py, and the FP6 GEMM with the
INT8 path's exact accumulators.
"""
import numpy as np


def test_e3m2_ocp_figures(oracle):
    vals = np.array([oracle.e3m2_to_f32(b) for b in range(64)], dtype=np.float64)
    assert np.all(np.isfinite(vals))
    assert vals[0b011111] == 28.0  # largest normal
    assert vals[0b000100] == 0.25  # smallest normal
    assert vals[0b000001] == 0.0625  # smallest subnormal
    assert np.all(np.diff(vals[:32]) > 0)  # magnitudes increase with the code
    assert np.array_equal(vals[32:], -vals[:32])


def test_integer_codes_round_trip(oracle):
    for v in range(-8, 9):
        bits = oracle.e3m2_of_int(v)
        assert bits < 64
        assert oracle.e3m2_to_f32(bits) == float(v)
    assert oracle.e3m2_of_int(9) == 255  # 9 = 1.125 x 8 needs a third mantissa bit


def test_chunk_layout_unpacks(oracle):
    rng = np.random.default_rng(11)
    codes = rng.integers(-8, 8, size=(7, 64)).astype(np.int8)
    chunks = oracle.fp6_chunks(codes)
    assert chunks.shape == codes.shape
    flat = chunks.reshape(-1, 16)
    assert np.all(flat[:, 12:] == 0)
    bits = np.unpackbits(flat[:, :12], axis=1, bitorder="little")  # 96 bits a chunk, LSB first
    fields = bits.reshape(-1, 16, 6)
    f = (fields * (1 << np.arange(6))).sum(axis=2)
    decoded = np.array([[oracle.e3m2_to_f32(int(x)) for x in row] for row in f])
    assert np.array_equal(decoded.reshape(codes.shape), codes.astype(np.float64))
