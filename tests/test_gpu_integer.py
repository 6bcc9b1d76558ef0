"""GPU parity of the Integer strategy (QuantMatMul.cs:186-287, IntegerDot.cs)
through the C ABI, against the oracle.

Activation quantization and the integer products are bitwise equal to the
oracle: the block dots are exact int32 sums and every float step (scale
product, scaled sum, block-ascending accumulation, the Q5_1 offset term) is
the same operation in the same order.  Against the float path the reference's
own bounds apply (IntegerDotTests.cs:52-101).
"""
import ctypes

import numpy as np
import pytest

import jev
from oracle import oracle
from test_oracle_integer import _exact_case, integer_vs_float, reference_test_weights

pytestmark = pytest.mark.gpu
TYPES = [jev.TYPE_Q8_0, jev.TYPE_Q4_0, jev.TYPE_Q5_1]


@pytest.fixture
def integer(gpu):
    prev = jev.get_matmul_strategy()
    jev.set_matmul_strategy(jev.MATMUL_INTEGER)
    try:
        yield
    finally:
        jev.set_matmul_strategy(prev)


def matmul_gpu(t, raw, rows, cols, x, tokens):
    y = np.empty(tokens * rows, np.float32)
    xx = np.ascontiguousarray(x, np.float32)
    b = np.ascontiguousarray(raw, dtype=np.uint8)
    F = ctypes.POINTER(ctypes.c_float)
    jev._lib.check(jev.lib().jev_matmul_q(t, b.ctypes.data_as(ctypes.c_void_p), rows, cols, xx.ctypes.data_as(F),
                                          tokens, y.ctypes.data_as(F)))
    return y.reshape(tokens, rows)


def test_strategy_switch(gpu):
    assert jev.get_matmul_strategy() == jev.MATMUL_AUTO  # QuantMatMul.cs:41
    with pytest.raises(jev.ArgumentError):
        jev.set_matmul_strategy(7)
    assert jev.get_matmul_strategy() == jev.MATMUL_AUTO


@pytest.mark.parametrize("n", [32, 1024, 3072, 9216])
def test_gpu_activation_quantization_bitwise(gpu, n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 10.0 ** rng.uniform(-6, 2, n // 32).repeat(32)).astype(np.float32)
    x[:32] = 0.0                              # an all-zero block
    if n >= 64:
        x[32:64] = 0.0
        x[32], x[33:37] = 127.0, [2.5, -2.5, 0.5, -1.5]  # exact ties, half away from zero
    got_q, got_s = jev.quantize_activations(x)
    want_q, want_s = oracle.quantize_activations(x)
    assert np.array_equal(got_q, want_q)
    assert np.array_equal(got_s.view(np.uint32), want_s.view(np.uint32))


def test_gpu_activation_round_trip_and_zero_block(gpu):
    # IntegerDotTests.cs:104-147 on the device's quantizer
    values = np.random.default_rng(11).uniform(-4, 4, 1024).astype(np.float32)
    q, _ = jev.quantize_activations(values)
    restored = oracle.dequantize(jev.TYPE_Q8_0, q, 1024)
    blockmax = np.abs(values).reshape(-1, 32).max(axis=1).repeat(32)
    assert float(np.max(np.abs(restored - values) / blockmax)) < 1.0 / 254 * 1.05
    z, zs = jev.quantize_activations(np.zeros(32, np.float32))
    assert not z.any() and not zs.any()
    with pytest.raises(jev.ArgumentError):
        jev.quantize_activations(np.zeros(40, np.float32))


SHAPES = [(96, 3072, 3), (128, 256, 1), (64, 4096, 6), (48, 1056, 17), (200, 512, 33), (3072, 3072, 256),
          (1024, 3072, 1), (384, 1088, 130)]


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("rows,cols,tokens", SHAPES)
def test_gpu_integer_matmul_bitwise_vs_oracle(integer, t, rows, cols, tokens):
    raw = jev.synth_tensor(f"i{rows}x{cols}", t, rows, cols, 0.02, seed=tokens)
    x = np.random.default_rng(rows + cols + tokens).standard_normal((tokens, cols)).astype(np.float32)
    want = oracle.matmul_integer(t, raw, rows, cols, x, tokens)
    got = matmul_gpu(t, raw, rows, cols, x, tokens)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (t, rows, cols, tokens)


@pytest.mark.parametrize("t", TYPES)
def test_gpu_integer_matmul_exact_inputs(integer, t):
    raw, x, want = _exact_case(t, 48, 1056, 5, seed=t)
    got = matmul_gpu(t, raw, 48, 1056, x, 5)
    assert np.array_equal(got.astype(np.float64), want)


@pytest.mark.parametrize("t", TYPES)
def test_gpu_integer_path_agrees_with_gpu_float_path(gpu, t):
    # IntegerDotTests.IntegerPathAgreesWithFloatPath (:52-101): both paths on the device
    def run(strategy):
        def fn(tt, raw, rows, cols, x, tokens):
            prev = jev.get_matmul_strategy()
            jev.set_matmul_strategy(strategy)
            try:
                return matmul_gpu(tt, raw, rows, cols, x, tokens)
            finally:
                jev.set_matmul_strategy(prev)
        return fn
    stats = [integer_vs_float(t, s, run(jev.MATMUL_INTEGER), run(jev.MATMUL_FLOAT)) for s in range(8)]
    assert max(r for r, _ in stats) < 0.01, stats
    assert abs(np.mean([b for _, b in stats])) < 2e-3, stats


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("rows,cols,tokens", [(3072, 3072, 256), (96, 3072, 3), (1024, 3072, 1)])
def test_gpu_resident_weight_integer_matches_hook_bitwise(integer, t, rows, cols, tokens):
    import torch
    raw = reference_test_weights(t, rows, cols, 3)
    x = np.random.default_rng(4).uniform(-1, 1, (tokens, cols)).astype(np.float32)
    w = jev.QuantWeight(t, rows, cols, raw)
    dx = torch.from_numpy(x).to("cuda:0")
    dy = torch.empty((tokens, rows), dtype=torch.float32, device="cuda:0")
    w.matmul_device(dx.data_ptr(), tokens, dy.data_ptr())
    w.sync()
    got = dy.cpu().numpy()
    w.close()
    want = matmul_gpu(t, raw, rows, cols, x, tokens)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("t", TYPES)
def test_gpu_integer_unaligned_input_gives_the_same_bits(integer, t):
    # x one float past a 16-byte boundary takes the one-element activation
    # quantizer instead of the four-element one: the same quants, scales and
    # sums, so the same outputs
    import torch
    rows, cols, tokens = 384, 1088, 130
    raw = reference_test_weights(t, rows, cols, 5)
    x = np.random.default_rng(6).uniform(-1, 1, (tokens, cols)).astype(np.float32)
    w = jev.QuantWeight(t, rows, cols, raw)
    bx = torch.from_numpy(np.concatenate([np.zeros(1, np.float32), x.reshape(-1)])).to("cuda:0")
    dx = torch.from_numpy(x).to("cuda:0")
    dy0 = torch.empty((tokens, rows), dtype=torch.float32, device="cuda:0")
    dy1 = torch.empty((tokens, rows), dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    assert bx.data_ptr() % 16 == 0
    w.matmul_device(bx.data_ptr() + 4, tokens, dy0.data_ptr())
    w.matmul_device(dx.data_ptr(), tokens, dy1.data_ptr())
    w.sync()
    got, want = dy0.cpu().numpy(), dy1.cpu().numpy()
    w.close()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(want.view(np.uint32), oracle.matmul_integer(t, raw, rows, cols, x, tokens).view(np.uint32))
