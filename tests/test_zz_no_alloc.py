"""jev_matmul_device_noalloc: the resident-weight matmul with its scratch in the
library's static device array instead of allocations.  Through the C ABI it must
give the same bits as jev_matmul_device (the same kernels), on two calls in a
row where the second is smaller (the array keeps the first call's contents),
for the GEMM, the GEMV, a Q5_1 weight (block sums) and the integer strategy,
and refuse a call whose scratch would not fit before any kernel runs."""
import numpy as np
import pytest

import jev

pytestmark = pytest.mark.gpu


def _run(w, fn, x, rows):
    import torch
    dx = torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0")
    dy = torch.full((x.shape[0], rows), float("nan"), dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    fn(dx.data_ptr(), x.shape[0], dy.data_ptr())
    w.sync()
    return dy.cpu().numpy()


@pytest.mark.parametrize("t,rows,cols,first,second", [
    (jev.TYPE_Q8_0, 3072, 3072, 256, 100),   # the single-matmul benchmark shape, K split in 4
    (jev.TYPE_Q5_1, 3072, 3072, 256, 17),
    (jev.TYPE_Q4_0, 1024, 3072, 64, 1),      # GEMM, then the one-token GEMV
    (jev.TYPE_Q8_0, 9216, 3072, 40, 2),
])
@pytest.mark.parametrize("strategy", [jev.MATMUL_FLOAT, jev.MATMUL_INTEGER])
def test_noalloc_equals_the_allocating_entry_point(gpu, t, rows, cols, first, second, strategy):
    raw = jev.synth_tensor(f"na{rows}x{cols}", t, rows, cols, 0.02, seed=9)
    rng = np.random.default_rng(first + second)
    xs = [rng.standard_normal((n, cols)).astype(np.float32) for n in (first, second)]
    w = jev.QuantWeight(t, rows, cols, raw)
    jev.set_matmul_strategy(strategy)
    try:
        got = [_run(w, w.matmul_device_noalloc, x, rows) for x in xs]  # two calls in a row, smaller second
        want = [_run(w, w.matmul_device, x, rows) for x in xs]
    finally:
        jev.set_matmul_strategy(jev.MATMUL_AUTO)
        w.close()
    for g, e in zip(got, want):
        assert np.all(np.isfinite(e))
        assert np.array_equal(g, e)


def test_noalloc_refuses_a_call_beyond_its_scratch(gpu):
    import torch
    raw = jev.synth_tensor("na_big", jev.TYPE_Q8_0, 3072, 3072, 0.02, seed=9)
    w = jev.QuantWeight(jev.TYPE_Q8_0, 3072, 3072, raw)
    dx = torch.zeros((700, 3072), dtype=torch.float32, device="cuda:0")
    dy = torch.zeros((700, 3072), dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    try:
        # 700 tokens: K-split partials alone are 700 x 3072 x 4 splits x 4 B = 34 MB
        with pytest.raises(jev.ArgumentError, match="scratch"):
            w.matmul_device_noalloc(dx.data_ptr(), 700, dy.data_ptr())
        w.sync()
        assert not dy.any()  # nothing ran
    finally:
        w.close()
