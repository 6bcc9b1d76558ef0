"""Pins the oracle's kernels against definitions, closed forms and the
reference's own invariants (PanelGemmTests.cs, KernelTests.cs,
AttentionKernelTests.cs, RopeAndCacheTests.cs).  Expectations are computed in
float64 by independent numpy formulations, never by restating the oracle's
loops.
"""
import math

import numpy as np
import pytest

import jev
from helpers import worst_close
from oracle import oracle


def q8(rows, cols, seed):
    rng = np.random.default_rng(seed)
    w = rng.uniform(-1, 1, (rows, cols)).astype(np.float32)
    raw = jev.quantize(w, jev.TYPE_Q8_0)
    return raw, oracle.dequantize(jev.TYPE_Q8_0, raw, rows * cols).reshape(rows, cols)


# PanelGemmTests.cs:38-59 shapes (rows, cols, tokens): across KBlock = 2048 and FFN width 9216.
@pytest.mark.parametrize("rows,cols,tokens", [(128, 256, 1), (64, 3072, 5), (128, 3072, 13), (64, 4096, 6), (64, 9216, 7)])
def test_matmul_matches_definition(rows, cols, tokens):
    raw, w = q8(rows, cols, rows + cols + tokens)
    x = np.random.default_rng(tokens).uniform(-1, 1, (tokens, cols)).astype(np.float32)
    y = oracle.matmul(jev.TYPE_Q8_0, raw, rows, cols, x, tokens)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    assert worst_close(ref, y) <= 1e-4


def test_panel_gemm_is_one_fma_chain_per_output():
    # The panel path (tokens >= 2) must equal a single fused chain over k
    # ascending, computed here with numpy float64 per step rounded to float32
    # through an exact fma emulation (float64 holds a float32 product exactly).
    rows, cols = 64, 96
    raw, w = q8(rows, cols, 5)
    x = np.random.default_rng(9).uniform(-2, 2, (3, cols)).astype(np.float32)
    y = oracle.matmul(jev.TYPE_Q8_0, raw, rows, cols, x, 3)
    acc = np.zeros((3, rows), np.float32)
    for k in range(cols):
        prod = x[:, k:k + 1].astype(np.float64) * w[:, k][None, :].astype(np.float64)
        acc = (acc.astype(np.float64) + prod).astype(np.float32)  # fma: one rounding of exact product + acc
    assert np.array_equal(acc, y)


def test_batch_invariance_bitwise():
    # A token's result does not depend on its batch (PanelGemmTests.cs:61-74).
    rows, cols = 128, 3072
    raw, _ = q8(rows, cols, 1)
    x = np.random.default_rng(2).uniform(-1, 1, (17, cols)).astype(np.float32)
    full = oracle.matmul(jev.TYPE_Q8_0, raw, rows, cols, x, 17)
    tail = oracle.matmul(jev.TYPE_Q8_0, raw, rows, cols, x[12:], 5)
    assert np.array_equal(full[12:], tail)


def test_threads_do_not_change_bits():
    # Fan-out invariance (PanelGemmTests.cs:76-89).
    rows, cols = 256, 1024
    raw, _ = q8(rows, cols, 4)
    x = np.random.default_rng(5).uniform(-1, 1, (9, cols)).astype(np.float32)
    oracle.set_threads(1)
    a = oracle.matmul(jev.TYPE_Q8_0, raw, rows, cols, x, 9)
    oracle.set_threads(0)
    b = oracle.matmul(jev.TYPE_Q8_0, raw, rows, cols, x, 9)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("t", [jev.TYPE_Q4_0, jev.TYPE_Q5_1, jev.TYPE_Q8_0])
def test_quantized_equals_dequantized_twin(t):
    # KernelTests.cs:232-270: the quantized product equals the product with the decoded weights.
    rows, cols = 64, 512
    w = np.random.default_rng(11).standard_normal((rows, cols)).astype(np.float32)
    raw = jev.quantize(w, t)
    deq = oracle.dequantize(t, raw, rows * cols).reshape(rows, cols)
    x = np.random.default_rng(12).uniform(-1, 1, (4, cols)).astype(np.float32)
    y = oracle.matmul(t, raw, rows, cols, x, 4)
    ref = x.astype(np.float64) @ deq.astype(np.float64).T
    assert worst_close(ref, y) <= 1e-5


LENGTHS = [1, 2, 3, 7, 8, 15, 16, 17, 31, 33, 64, 127, 3072, 9216]  # KernelTests.cs:26-104


@pytest.mark.parametrize("n", LENGTHS)
def test_rmsnorm_definition(n):
    rng = np.random.default_rng(n)
    x = rng.uniform(-1, 1, n).astype(np.float32)
    w = rng.uniform(-1, 1, n).astype(np.float32)
    y = oracle.rmsnorm(x, w, 1e-5)
    xd = x.astype(np.float64)
    ref = xd / math.sqrt((xd * xd).mean() + 1e-5) * w
    assert worst_close(ref, y) <= 1e-5


@pytest.mark.parametrize("n", LENGTHS)
def test_softmax_definition(n):
    x = np.random.default_rng(n + 1).uniform(-8, 8, n).astype(np.float32)
    y = oracle.softmax(x)
    e = np.exp(x.astype(np.float64) - x.max())
    assert worst_close(e / e.sum(), y) <= 1e-6


def test_softmax_large_scores_do_not_overflow():
    y = oracle.softmax(np.array([90.0, 95.0, 100.0], np.float32))
    assert np.all(np.isfinite(y)) and abs(y.sum() - 1) < 1e-6


def test_softmax_fully_masked_row_is_uniform():
    # KernelTests.cs:138-146
    y = oracle.softmax(np.full(4, -np.inf, np.float32))
    assert np.array_equal(y, np.full(4, 0.25, np.float32))


@pytest.mark.parametrize("n", LENGTHS)
def test_swiglu_definition(n):
    rng = np.random.default_rng(n + 2)
    g = rng.uniform(-4, 4, n).astype(np.float32)
    u = rng.uniform(-4, 4, n).astype(np.float32)
    y = oracle.swiglu(g, u)
    gd, ud = g.astype(np.float64), u.astype(np.float64)
    assert worst_close(gd / (1 + np.exp(-gd)) * ud, y) <= 1e-5


@pytest.mark.parametrize("length", [1, 15, 17, 64, 211])
def test_attention_matches_brute_force(length):
    # AttentionKernelTests.cs:24-58 lengths; causal over `length` keys.
    rng = np.random.default_rng(length)
    k = rng.uniform(-1, 1, (length, 128)).astype(np.float32)
    v = rng.uniform(-1, 1, (length, 128)).astype(np.float32)
    q = rng.uniform(-1, 1, 128).astype(np.float32)
    scale = 1 / math.sqrt(128)
    out = oracle.attend(q, k, v, 0, 0, 0, length - 1, scale)
    s = (k.astype(np.float64) @ q) * scale
    p = np.exp(s - s.max())
    p /= p.sum()
    assert worst_close(p @ v, out) <= 1e-4


def test_attention_tree_visibility_and_range_start_invariance():
    # Keys [shared_lo, shared_hi) and [segment, slot] only; and a key's score
    # does not depend on where its range starts (AttentionKernelTests.cs:61-77):
    # a branch laid out after other branches equals the same branch laid
    # out right after the trunk.
    rng = np.random.default_rng(7)
    n = 40
    k = rng.uniform(-1, 1, (n, 128)).astype(np.float32)
    v = rng.uniform(-1, 1, (n, 128)).astype(np.float32)
    q = rng.uniform(-1, 1, 128).astype(np.float32)
    scale = 1 / math.sqrt(128)
    # trunk [2, 12), branch at [30, 34], query at slot 34
    out = oracle.attend(q, k, v, 2, 12, 30, 34, scale)
    vis = list(range(2, 12)) + list(range(30, 35))
    s = (k[vis].astype(np.float64) @ q) * scale
    p = np.exp(s - s.max())
    p /= p.sum()
    assert worst_close(p @ v[vis], out) <= 1e-5
    # same visible rows packed contiguously: bit-identical
    k2, v2 = k[vis], v[vis]
    out2 = oracle.attend(q, k2, v2, 0, 10, 10, 14, scale)
    assert np.array_equal(out, out2)


def test_rope_properties():
    cfg = jev.ModelConfig(n_layers=1, hidden=256, n_heads=2, n_kv_heads=1, ffn=512, vocab=64)
    freqs, mscale = oracle.rope_freqs(cfg)
    assert mscale == 1.0 and freqs[0] == 1.0
    ref = 1.0 / np.power(np.float64(1e6), 2 * np.arange(64) / 128)
    assert np.allclose(freqs, ref, rtol=1e-6)
    x = np.random.default_rng(1).uniform(-1, 1, 256).astype(np.float32)
    # identity at position 0 (RopeAndCacheTests.cs:49-60)
    assert np.array_equal(oracle.rope_apply(freqs, mscale, x, 2, 128, 0), x)
    # norm preserving, adjacent pairs rotated by position * freq, heads independent
    for pos in (1, 17, 4095):
        y = oracle.rope_apply(freqs, mscale, x, 2, 128, pos).astype(np.float64)
        xd = x.astype(np.float64).reshape(2, 64, 2)
        th = (np.float32(pos) * freqs).astype(np.float64)  # the angle is a float product (Rope.cs:120)
        c, s = np.cos(th), np.sin(th)
        ref = np.stack([xd[..., 0] * c - xd[..., 1] * s, xd[..., 0] * s + xd[..., 1] * c], -1).reshape(-1)
        assert np.max(np.abs(y - ref)) < 1e-5
        assert abs(np.linalg.norm(y) - np.linalg.norm(x)) < 1e-4


def test_yarn_ramp_ends():
    # With YaRN active, the lowest pairs keep the extrapolated frequency and
    # the highest take the interpolated one (RopeAndCacheTests.cs:100-142).
    cfg = jev.ModelConfig(n_layers=1, hidden=256, n_heads=2, n_kv_heads=1, ffn=512, vocab=64,
                          rope_scale_factor=16.0, rope_scaling_yarn=1, rope_original_context=16384,
                          yarn_mscale_all_dim=1.0, yarn_mscale=1.0)
    freqs, mscale = oracle.rope_freqs(cfg)
    ext = 1.0 / np.power(1e6, 2 * np.arange(64) / 128)
    assert abs(freqs[0] - ext[0]) < 1e-7
    assert abs(freqs[-1] - ext[-1] / 16) / (ext[-1] / 16) < 1e-5
    assert mscale == 1.0


def test_layout_tree_closed_form():
    # TokenLayout.Tree (MinistralModel.cs:720-745): trunk of 3 after 5 cached, branches of 2 and 3.
    slot, pos, sh, seg, outs, end = oracle.layout_tree(5, 3, [3, 5], 8)
    assert list(slot) == list(range(5, 13))
    assert list(pos) == [5, 6, 7, 8, 9, 8, 9, 10]
    assert list(sh) == [5, 5, 5, 8, 8, 8, 8, 8]
    assert list(seg) == [5, 5, 5, 8, 8, 10, 10, 10]
    assert list(outs) == [4, 7] and end == 13


def test_layout_rows_closed_form():
    slot, pos, sh, seg, outs, end = oracle.layout_rows(4, [10, 20], [2, 0], [1, 3])
    assert list(slot) == [12, 20, 21, 22]
    assert list(pos) == [6, 4, 5, 6]
    assert list(sh) == [4, 4, 4, 4] and list(seg) == [10, 20, 20, 20]
    assert list(outs) == [0, 3] and end == 23


def test_margins_and_probabilities():
    v = np.array([[2.0, 1.0, 0.5, 0.0], [0.0, 3.0, 1.0, 0.5]], np.float32)  # yes rows 0-1, no rows 2-3
    m, p = oracle.margins(v, 2, 2, 1.0)
    assert np.allclose(m, [1.5, 2.0])
    e = np.exp(np.array([1.5, 2.0]) - 2.0)
    assert np.allclose(p, e / e.sum(), rtol=1e-6)
    jm, jp = jev.margins(v, 2, 2, 1.0)
    assert np.array_equal(jm, m) and np.allclose(jp, p, rtol=1e-6)


@pytest.mark.skipif(oracle.vector_bits() != 512, reason="the host has no AVX-512F")
@pytest.mark.parametrize("t", [jev.TYPE_Q4_0, jev.TYPE_Q5_1, jev.TYPE_Q8_0])
def test_panel_tile_widths_give_the_same_bits(t):
    # PanelGemm.VectorBits (PanelGemm.cs:50-63): the 512- and 256-bit tiles run
    # the same fused chain per output, so the oracle's CPU baseline on an
    # AVX-512 host computes exactly what the 256-bit path computes
    rows, cols, tokens = 128, 2304, 13  # two K blocks, a six-token remainder of 1
    raw = jev.synth_tensor("widths", t, rows, cols)
    x = np.random.default_rng(5).standard_normal((tokens, cols)).astype(np.float32)
    try:
        oracle.set_vector_bits(256)
        narrow = oracle.matmul(t, raw, rows, cols, x, tokens)
        oracle.set_vector_bits(512)
        wide = oracle.matmul(t, raw, rows, cols, x, tokens)
    finally:
        oracle.set_vector_bits(0)
    assert np.array_equal(narrow.view(np.uint32), wide.view(np.uint32))
