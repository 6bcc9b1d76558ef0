"""GPU parity of the HIP kernels through the C ABI test hooks, against the
oracle and the golden fixtures.  Tolerances: dequantisation bit-exact; the
quantized products at Numeric.Close 1e-4 (the bar of PanelGemmTests.cs:38-59)
against the oracle's float32 chain; batch invariance bitwise.
"""
import numpy as np
import pytest

import jev
from helpers import quant_fixtures, worst_close
from oracle import oracle

pytestmark = pytest.mark.gpu
FIX = quant_fixtures()


def dequant_gpu(t, raw, count):
    import ctypes
    out = np.empty(count, np.float32)
    b = np.ascontiguousarray(raw, dtype=np.uint8)
    jev._lib.check(jev.lib().jev_dequantize(t, b.ctypes.data_as(ctypes.c_void_p), b.nbytes,
                                            out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), count))
    return out


def matmul_gpu(t, raw, rows, cols, x, tokens):
    import ctypes
    y = np.empty(tokens * rows, np.float32)
    xx = np.ascontiguousarray(x, np.float32)
    b = np.ascontiguousarray(raw, dtype=np.uint8)
    F = ctypes.POINTER(ctypes.c_float)
    jev._lib.check(jev.lib().jev_matmul_q(t, b.ctypes.data_as(ctypes.c_void_p), rows, cols, xx.ctypes.data_as(F),
                                          tokens, y.ctypes.data_as(F)))
    return y.reshape(tokens, rows)


@pytest.mark.parametrize("name", ["Q4_0", "Q5_1", "Q8_0"])
@pytest.mark.parametrize("kind", ["quantized", "synthetic"])
def test_gpu_dequant_fixture_bit_exact(gpu, name, kind):
    t, entry = FIX[name]
    raw, expected = entry[kind]
    got = dequant_gpu(t, raw, expected.size)
    assert np.array_equal(got.view(np.uint32), expected.view(np.uint32))


@pytest.mark.parametrize("t", [jev.TYPE_Q4_0, jev.TYPE_Q5_1, jev.TYPE_Q8_0])
def test_gpu_dequant_random_blocks_bit_exact(gpu, t):
    # Random bytes with finite fp16 scales: the whole encoding space.
    rng = np.random.default_rng(t)
    ts = {2: 18, 7: 24, 8: 34}[t]
    raw = rng.integers(0, 256, size=(4096, ts), dtype=np.uint8)
    raw[:, 1] &= 0x3B  # keep d (and m) finite and moderate
    if t == jev.TYPE_Q5_1:
        raw[:, 3] &= 0x3B
    raw = raw.reshape(-1)
    exp = oracle.dequantize(t, raw, 4096 * 32)
    got = dequant_gpu(t, raw, 4096 * 32)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


SHAPES = [(128, 256, 1), (64, 3072, 5), (128, 3072, 13), (64, 4096, 6), (64, 9216, 7), (256, 512, 2),
          (384, 1024, 130), (3072, 3072, 256), (1024, 3072, 1), (384, 1088, 700), (200, 512, 513),
          (200, 1088, 250)]  # the last: 12-wave workgroups over a ragged N


@pytest.mark.parametrize("t", [jev.TYPE_Q4_0, jev.TYPE_Q5_1, jev.TYPE_Q8_0])
@pytest.mark.parametrize("rows,cols,tokens", SHAPES)
def test_gpu_matmul_matches_oracle(gpu, t, rows, cols, tokens):
    rng = np.random.default_rng(rows * 7 + cols + tokens)
    raw = jev.synth_tensor(f"w{rows}x{cols}", t, rows, cols, 0.02, seed=tokens)
    x = rng.standard_normal((tokens, cols)).astype(np.float32)
    exp = oracle.matmul(t, raw, rows, cols, x, tokens)
    got = matmul_gpu(t, raw, rows, cols, x, tokens)
    assert worst_close(exp, got) <= 1e-4, (t, rows, cols, tokens)


@pytest.mark.parametrize("t", [jev.TYPE_Q4_0, jev.TYPE_Q5_1, jev.TYPE_Q8_0])
@pytest.mark.parametrize("rows,cols", [(384, 3072), (200, 1056)])
def test_gpu_matmul_batch_invariance_bitwise(gpu, t, rows, cols):
    # A token's result does not depend on its batch (PanelGemmTests.cs:61-74),
    # across the M tile boundary (128) too.
    # Small-M and large-M calls take different tile shapes; bits must not move.
    # 200 x 1056: a weight that ends inside a 32-row group, 33 quant blocks
    # (an odd block count in the last K split).
    raw = jev.synth_tensor("inv", t, rows, cols)
    x = np.random.default_rng(1).standard_normal((700, cols)).astype(np.float32)
    full = matmul_gpu(t, raw, rows, cols, x, 700)
    mid = matmul_gpu(t, raw, rows, cols, x[:300], 300)
    part = matmul_gpu(t, raw, rows, cols, x[120:137], 17)
    assert np.array_equal(full[:300], mid)
    assert np.array_equal(full[120:137], part)
    # 225..256 rows take the 12-wave workgroups
    for lo, n in ((0, 256), (300, 240)):
        assert np.array_equal(full[lo:lo + n], matmul_gpu(t, raw, rows, cols, x[lo:lo + n], n)), n
    # 2..16 tokens take the one-wave-per-row-group kernel: the same chain per output
    for lo, n in ((0, 2), (33, 9), (684, 16)):
        assert np.array_equal(full[lo:lo + n], matmul_gpu(t, raw, rows, cols, x[lo:lo + n], n)), n
    again = matmul_gpu(t, raw, rows, cols, x, 700)
    assert np.array_equal(full, again)


def test_gpu_matmul_rejects_bad_shapes(gpu):
    raw = jev.synth_tensor("bad", jev.TYPE_Q8_0, 64, 64)
    with pytest.raises(jev.ArgumentError):
        matmul_gpu(jev.TYPE_Q8_0, raw, 64, 48, np.zeros((2, 48), np.float32), 2)


@pytest.mark.parametrize("t", [jev.TYPE_Q4_0, jev.TYPE_Q5_1, jev.TYPE_Q8_0])
@pytest.mark.parametrize("rows,cols,tokens", [(3072, 3072, 256), (384, 1088, 700), (1024, 3072, 1), (200, 512, 3)])
def test_gpu_resident_weight_matches_test_hook_bitwise(gpu, t, rows, cols, tokens):
    # The resident-weight seam (jev_weight_*) runs the same kernels and K
    # splits as the upload-per-call hook, so the bits agree; the hook itself
    # is pinned to the oracle above.
    import torch
    raw = jev.synth_tensor(f"res{rows}x{cols}", t, rows, cols, 0.02, seed=5)
    x = np.random.default_rng(7).standard_normal((tokens, cols)).astype(np.float32)
    w = jev.QuantWeight(t, rows, cols, raw)
    dx = torch.from_numpy(x).to("cuda:0")
    dy = torch.empty((tokens, rows), dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    w.matmul_device(dx.data_ptr(), tokens, dy.data_ptr())
    w.sync()
    got = dy.cpu().numpy()
    w.close()
    assert np.array_equal(got, matmul_gpu(t, raw, rows, cols, x, tokens))
    if rows * cols * tokens <= 384 * 1088 * 700:
        assert worst_close(oracle.matmul(t, raw, rows, cols, x, tokens), got) <= 1e-4


@pytest.mark.parametrize("t", [jev.TYPE_Q4_0, jev.TYPE_Q5_1, jev.TYPE_Q8_0])
def test_gpu_resident_weight_unaligned_buffers_give_the_same_bits(gpu, t):
    # x and y one float past a 16-byte boundary take the one-element split and
    # partial-sum kernels instead of the vector ones: the same arithmetic
    import torch
    rows, cols, tokens = 384, 1088, 130
    raw = jev.synth_tensor(f"una{rows}x{cols}", t, rows, cols, 0.02, seed=3)
    x = np.random.default_rng(5).standard_normal((tokens, cols)).astype(np.float32)
    w = jev.QuantWeight(t, rows, cols, raw)
    bx = torch.from_numpy(np.concatenate([np.zeros(1, np.float32), x.reshape(-1)])).to("cuda:0")
    by = torch.zeros(tokens * rows + 1, dtype=torch.float32, device="cuda:0")
    dx = torch.from_numpy(x).to("cuda:0")
    dy = torch.empty((tokens, rows), dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    assert bx.data_ptr() % 16 == 0 and by.data_ptr() % 16 == 0
    w.matmul_device(bx.data_ptr() + 4, tokens, by.data_ptr() + 4)
    w.matmul_device(dx.data_ptr(), tokens, dy.data_ptr())
    w.sync()
    got = by.cpu().numpy()
    want = dy.cpu().numpy()
    w.close()
    assert got[0] == 0.0
    assert np.array_equal(got[1:].reshape(tokens, rows), want)


@pytest.mark.parametrize("t", [jev.TYPE_Q4_0, jev.TYPE_Q5_1, jev.TYPE_Q8_0])
@pytest.mark.parametrize("cols", [4096, 4128])
def test_gpu_folded_k_splits_equal_the_summed_partials_bitwise(gpu, t, cols):
    # From 8192 rows the resident-weight seam's GEMM walks its four K-split
    # ranges in one workgroup and stores their sum in split order (Q8_0, Q4_0);
    # the test hook keeps four partial buffers and sums them after.  Same bits,
    # and each row as it comes out of a small batch.  4128 columns: 129 quant
    # blocks, a short last range ending in a half stage.
    import torch
    rows, tokens = 3072, 8200
    raw = jev.synth_tensor(f"fold{cols}", t, rows, cols, 0.02, seed=9)
    x = np.random.default_rng(11).standard_normal((tokens, cols)).astype(np.float32)
    w = jev.QuantWeight(t, rows, cols, raw)
    dx = torch.from_numpy(x).to("cuda:0")
    dy = torch.empty((tokens, rows), dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    w.matmul_device(dx.data_ptr(), tokens, dy.data_ptr())
    w.sync()
    got = dy.cpu().numpy()
    w.close()
    assert np.array_equal(got, matmul_gpu(t, raw, rows, cols, x, tokens))
    assert np.array_equal(got[8000:8017], matmul_gpu(t, raw, rows, cols, x[8000:8017], 17))
