"""The synthetic-model quantizers (jev_quantize, host code of libjev) against
the reference's fixture bytes.

The reference's fixture generator (tools/gen_quant_fixtures.py) draws its
inputs from numpy.random.default_rng(20260806) in a fixed order: 64 normals
each for F32, F16 and BF16, then per block type (Q4_0, Q4_1, Q5_0, Q5_1, Q8_0
in that order) 256 normals * 0.35 for the "quantized" case and random block
bytes for the "synthetic" case, dropping blocks that decode non-finite or
above 1e6.  Replaying that order regenerates the exact quantizer inputs, so
the ggml-reference quantizers must reproduce the fixture's "quantized" bytes
bit for bit.  The replay is itself checked: its synthetic blocks must equal
the fixture's synthetic bytes.
"""
import numpy as np
import pytest

import jev
from helpers import quant_fixtures

FIX = quant_fixtures()


def _h(b):
    return np.frombuffer(np.asarray(b, np.uint8).tobytes(), np.float16).astype(np.float32)


def _nib(qs):
    return np.concatenate([(qs & 15), (qs >> 4)]).astype(np.float32)


def _fifth(qh):
    return np.array([(qh >> j) & 1 for j in range(32)], np.float32) * 16


# numpy statements of the block decoders, only to replay the fixture's
# rejection of non-finite / huge random blocks.
DECODE = {
    "Q4_0": (18, lambda r: _h(r[0:2]) * (_nib(r[2:18]) - 8)),
    "Q4_1": (20, lambda r: _h(r[0:2]) * _nib(r[4:20]) + _h(r[2:4])),
    "Q5_0": (22, lambda r: _h(r[0:2]) * (_nib(r[6:22]) + _fifth(int(np.frombuffer(r[2:6].tobytes(), np.uint32)[0])) - 16)),
    "Q5_1": (24, lambda r: _h(r[0:2]) * (_nib(r[8:24]) + _fifth(int(np.frombuffer(r[4:8].tobytes(), np.uint32)[0])))
             + _h(r[2:4])),
    "Q8_0": (34, lambda r: _h(r[0:2]) * r[2:34].view(np.int8).astype(np.float32)),
}


def replay():
    rng = np.random.default_rng(20260806)
    for _ in range(3):
        rng.standard_normal(64).astype(np.float32)
    sources, synth = {}, {}
    for name in ("Q4_0", "Q4_1", "Q5_0", "Q5_1", "Q8_0"):
        ts, dec = DECODE[name]
        sources[name] = rng.standard_normal(8 * 32).astype(np.float32) * 0.35
        kept = []
        for _ in range(200):
            if len(kept) >= 8:
                break
            raw = rng.integers(0, 256, size=ts, dtype=np.uint8)
            with np.errstate(all="ignore"):
                v = dec(raw)
            if not np.all(np.isfinite(v)) or np.max(np.abs(v)) > 1e6:
                continue
            kept.append(raw)
        synth[name] = np.concatenate(kept)
    return sources, synth


SOURCES, SYNTH = replay()


@pytest.mark.parametrize("name", ["Q4_0", "Q5_1", "Q8_0"])
def test_replay_is_in_step_with_the_fixture(name):
    _, entry = FIX[name]
    assert np.array_equal(SYNTH[name], entry["synthetic"][0])


@pytest.mark.parametrize("name", ["Q4_0", "Q5_1", "Q8_0"])
def test_quantizer_reproduces_fixture_bytes(name):
    t, entry = FIX[name]
    got = jev.quantize(SOURCES[name], t)
    assert np.array_equal(got, entry["quantized"][0])


def test_quantizer_round_trip_error_is_bounded():
    x = np.random.default_rng(3).standard_normal(32 * 64).astype(np.float32)
    from oracle import oracle
    # half a quantization step, except Q4_0, whose step is amax/8 and whose
    # top code (+8) is clamped to 7: up to one full step there.
    for t, tol in ((jev.TYPE_Q8_0, 0.5 / 127), (jev.TYPE_Q4_0, 1 / 8), (jev.TYPE_Q5_1, 0.5 / 31)):
        y = oracle.dequantize(t, jev.quantize(x, t), x.size)
        amax = np.abs(x.reshape(-1, 32)).max(1, keepdims=True)
        rng_ = (x.reshape(-1, 32).max(1, keepdims=True) - x.reshape(-1, 32).min(1, keepdims=True))
        scale = rng_ if t == jev.TYPE_Q5_1 else amax
        assert np.all(np.abs(y.reshape(-1, 32) - x.reshape(-1, 32)) <= scale * tol + 1e-3 * scale)


def test_synth_is_deterministic_and_thread_independent():
    import ctypes
    a = jev.synth_tensor("blk.0.attn_q.weight", jev.TYPE_Q8_0, 256, 512)
    b = np.empty_like(a)
    import zlib
    jev.lib().jev_synth_tensor(jev.SEED, zlib.crc32(b"blk.0.attn_q.weight"), jev.TYPE_Q8_0, 256, 512, 0.02,
                               b.ctypes.data_as(ctypes.c_void_p), b.nbytes, 1)
    assert np.array_equal(a, b)
    c = jev.synth_tensor("blk.0.attn_k.weight", jev.TYPE_Q8_0, 256, 512)
    assert not np.array_equal(a, c)


def test_synth_distribution():
    v = jev.synth_tensor("w", jev.TYPE_F32, 512, 1024).view(np.float32)
    assert abs(v.mean()) < 2e-4 and abs(v.std() - 0.02) < 2e-4
