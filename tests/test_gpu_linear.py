"""Sparse Linear on the GPU (sf_linear_prescan / sf_linear_sparse through
Kernels.linear.sparse_linear_forward and SparseLinear).

Bar: row bitmap and chunk flags bit-exact against oracle/linear.py; fp32
outputs within 1e-4 abs + 1e-4 rel of float64 F.linear on the activity-
masked input; fp16/bf16 within 1e-2; bit-identical repeats."""

import numpy as np
import pytest
import torch

from oracle import linear as olin
from sparseflow_amd import _lib
from sparseflow_amd.Kernels.linear import sparse_linear_forward
from sparseflow_amd.Ops.sparse_linear import SparseLinear
from tests.gpu_helpers import DEV, announce, close, native_loaded, spikes

pytestmark = pytest.mark.gpu

FP32_TOL = dict(atol=1e-4, rtol=1e-4)


def _w(c_out, k, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(c_out, k, generator=g) * (1.0 / k) ** 0.5


def _run(x, w, b, **kw):
    torch.cuda.synchronize()
    _lib.timing_reset()
    _lib.timing_enable(True)
    try:
        y = sparse_linear_forward(x, w, b, **kw)[0]
        torch.cuda.synchronize()
        stats = _lib.timing_collect()
    finally:
        _lib.timing_enable(False)
    return y, {k: c for k, (c, _) in stats.items() if c > 0}


CASES = [
    (1, 1, 4), (17, 33, 12), (64, 64, 64), (100, 100, 68), (130, 130, 8), (1000, 384, 384),
    (4096, 1536, 384), (512, 2048, 1000), (3, 4100, 16),
]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("density", [0.0, 0.1, 0.5])
@pytest.mark.parametrize("kernel", ["walk", "mfma", "mfma_bits"])
def test_linear_fp32_matches_dense(case, density, kernel):
    m, k, co = case
    announce(f"linear {kernel} {case} p={density}")
    x = spikes((m, k), density, seed=m + k)
    w = _w(co, k, seed=co)
    b = torch.randn(co, generator=torch.Generator().manual_seed(5)) * 0.1
    y, kernels = _run(x.to(DEV), w.to(DEV), b.to(DEV), kernel=kernel)
    if kernel == "walk":
        assert "linear_flat" in kernels and "prescan_rows" in kernels, kernels
    else:
        assert set(kernels) == ({"prescan_rows", "linear_mfma"} if kernel == "mfma_bits" else {"linear_mfma"}), kernels
    ok, err, _ = close(y, olin.linear_ref(x, w, b), **FP32_TOL)
    assert ok, f"max abs err {err}"
    assert native_loaded()


@pytest.mark.parametrize("m,k", [(5, 20), (40, 64), (33, 100), (300, 384), (17, 1536), (33, 37), (9, 258),
                                 (64, 260)])
@pytest.mark.parametrize("aligned", [True, False])
def test_row_bitmap_and_flags_bit_exact(m, k, aligned):
    # f32 rows with k % 4 == 0 at a 16-byte aligned address take the 16-byte
    # load kernel, the rest the per-element one: both bit-exact.
    announce(f"linear bitmap {m}x{k} aligned={aligned}")
    x = spikes((m, k), 0.2, seed=k)
    x[m // 2, k // 3] = 2.5          # non-binary chunk
    x[0, 0] = 4e-7                   # below the threshold
    if aligned:
        xd = x.to(DEV)
    else:  # one element past a 16-byte boundary
        buf = torch.zeros(m * k + 1, device=DEV)
        buf[1:] = x.reshape(-1).to(DEV)
        xd = buf[1:].view(m, k)
    bits, flags = _lib.linear_prescan(xd, 1e-6)
    words = olin.linear_words_per_row(k)
    got = bits[: m * words].cpu().numpy().view(np.uint32).reshape(m, words)
    assert np.array_equal(got, olin.row_bitmap(x.numpy(), 1e-6))
    nb = flags[: -(-m // 16)].cpu().numpy() != 0
    assert np.array_equal(nb, olin.row_chunk_nonbinary(x.numpy()))


@pytest.mark.parametrize("kernel", ["walk", "mfma", "mfma_bits"])
def test_value_path_inputs(kernel):
    g = torch.Generator().manual_seed(7)
    x = spikes((256, 384), 0.1, seed=8)
    x[:64] = x[:64] * 2.0                                   # sums of two spike maps
    x[100:110] = x[100:110] * torch.randn(10, 384, generator=g)
    x[200, 5] = 3e-7                                        # below the activity threshold
    w = _w(384, 384, seed=9)
    announce(f"linear value path {kernel}")
    y, _ = _run(x.to(DEV), w.to(DEV), None, kernel=kernel)
    ok, err, _ = close(y, olin.linear_ref(x, w, None), **FP32_TOL)
    assert ok, f"max abs err {err}"


@pytest.mark.parametrize("kernel", ["mfma", "mfma_bits"])
def test_mfma_value_rows_only_where_x_is_not_binary(kernel):
    # One element that bf16 does not hold (0.3) in row 300.  The direct
    # kernel ("mfma") walks K a second time (x's bf16 lo part times W hi)
    # only in that 128-row block; the bitmap kernel ("mfma_bits") reads x instead
    # of the bitmap only in its 256-row block (the row chunk's non-binary
    # flag).  The result is exact to the fp32 bar and every other row equals
    # the all-spikes result bit for bit (binary rows of a value block too:
    # their third product adds zeros).
    x = spikes((1024, 384), 0.1, seed=31)
    w = _w(384, 384, seed=32)
    b = torch.randn(384, generator=torch.Generator().manual_seed(33)) * 0.1
    announce("linear mfma second walk")
    y0, _ = _run(x.to(DEV), w.to(DEV), b.to(DEV), kernel=kernel)
    x1 = x.clone()
    x1[300, 17] = 0.3                                       # 0.3 is not a bf16 value
    y1, _ = _run(x1.to(DEV), w.to(DEV), b.to(DEV), kernel=kernel)
    ok, err, _ = close(y1, olin.linear_ref(x1, w, b), **FP32_TOL)
    assert ok, f"max abs err {err}"
    ok, err, _ = close(y0, olin.linear_ref(x, w, b), **FP32_TOL)
    assert ok, f"max abs err {err}"
    assert torch.equal(y1[:300], y0[:300]) and torch.equal(y1[301:], y0[301:])
    assert not torch.equal(y1[300], y0[300])


@pytest.mark.parametrize("case", [(1000, 384, 384), (4096, 1536, 384), (777, 200, 1540)])
def test_mfma_bitmap_and_direct_kernels_agree_on_spikes(case):
    # Both accumulate, per 32-wide K step, x_hi @ W_hi then x_hi @ W_lo into
    # the same 16 x 16 tiles: on binary x they agree bit for bit.
    m, k, co = case
    announce(f"linear mfma bitmap vs direct {case}")
    x = spikes((m, k), 0.1, seed=m + k).to(DEV)
    w = _w(co, k, seed=co).to(DEV)
    b = (torch.randn(co, generator=torch.Generator().manual_seed(34)) * 0.1).to(DEV)
    yb, kb = _run(x, w, b, kernel="mfma_bits")
    yx, kx = _run(x, w, b, kernel="mfma")
    assert "prescan_rows" in kb and "prescan_rows" not in kx
    assert torch.equal(yb, yx)
    ok, err, _ = close(yb, olin.linear_ref(x.cpu(), w.cpu(), b.cpu()), **FP32_TOL)
    assert ok, f"max abs err {err}"


def test_mfma_bf16_split_keeps_fp32_accuracy():
    # Weights with full fp32 mantissas and large K: the hi + lo split keeps
    # the error far inside 1e-4 (one bf16 alone would not).
    g = torch.Generator().manual_seed(30)
    x = spikes((1024, 1536), 0.3, seed=31)
    w = torch.randn(384, 1536, generator=g) * 0.05
    announce("linear mfma accuracy")
    y, _ = _run(x.to(DEV), w.to(DEV), None, kernel="mfma")
    ref = olin.linear_ref(x, w, None)
    ok, err, _ = close(y, ref, **FP32_TOL)
    assert ok, f"max abs err {err}"
    assert err < 2e-5


@pytest.mark.parametrize("kernel", ["walk", "mfma", "mfma_bits"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_linear_half(dtype, kernel):
    x = spikes((512, 384), 0.1, seed=10)
    x[5] = x[5] * 0.5
    w = _w(384, 384, seed=11)
    b = torch.linspace(-0.5, 0.5, 384)
    announce(f"linear {dtype}")
    y, _ = _run(x.to(DEV, dtype), w.to(DEV), b.to(DEV), kernel=kernel)
    assert y.dtype == dtype
    ok, err, _ = close(y, olin.linear_ref(x.to(dtype).float(), w, b), atol=1e-2, rtol=1e-2)
    assert ok, f"max abs err {err}"
    y32, _ = _run(x.to(DEV, dtype), w.to(DEV), b.to(DEV), output_dtype=torch.float32, kernel=kernel)
    assert y32.dtype == torch.float32
    ok, err, _ = close(y32, olin.linear_ref(x.to(dtype).float(), w, b), **FP32_TOL)
    assert ok, f"max abs err {err}"


@pytest.mark.parametrize("kernel", ["walk", "mfma", "mfma_bits"])
def test_linear_deterministic_and_stats_path(kernel):
    x = spikes((2048, 384), 0.05, seed=12).to(DEV)
    w = _w(384, 384, seed=13).to(DEV)
    announce(f"linear determinism + stats {kernel}")
    y1, _ = _run(x, w, None, kernel=kernel)
    y2, _ = _run(x, w, None, kernel=kernel)
    assert torch.equal(y1, y2)
    res = sparse_linear_forward(x, w, None, return_ms=True, return_avg_active_ratio=True, return_tile_stats=True,
                                return_backend_meta=True, kernel=kernel)
    assert torch.equal(res[0], y1)
    assert 0.0 < res[2] <= 1.0 and res[3]["total_tiles"] == 16 and res[4]["backend"] == "sparse_hip"


def test_unsupported_c_out_falls_back_dense():
    x = spikes((64, 32), 0.1, seed=14)
    w = _w(6, 32, seed=15)
    res = sparse_linear_forward(x.to(DEV), w.to(DEV), None, return_backend_meta=True)
    assert res[2]["backend"] == "dense_fallback"
    ok, err, _ = close(res[0], olin.linear_ref(x, w, None), **FP32_TOL)
    assert ok


def test_sparse_linear_module_shapes():
    lin = torch.nn.Linear(384, 1536).to(DEV)
    sl = SparseLinear.from_dense(lin)
    x = spikes((4, 8, 49, 384), 0.1, seed=16).to(DEV)
    announce("SparseLinear module")
    y = sl(x)
    assert y.shape == (4, 8, 49, 1536)
    ok, err, _ = close(y, olin.linear_ref(x.cpu(), lin.weight, lin.bias), **FP32_TOL)
    assert ok, f"max abs err {err}"
    x5 = spikes((2, 3, 4, 4, 24), 0.2, seed=17).to(DEV)
    sl5 = SparseLinear.from_dense(torch.nn.Linear(4 * 4 * 24, 8).to(DEV))
    assert sl5(x5).shape == (2, 3, 8)


def _random_linear_cases(n, seed):
    g = torch.Generator().manual_seed(seed)
    out = []
    for _ in range(n):
        m = int(torch.randint(1, 3000, (1,), generator=g))
        k = int(torch.randint(1, 1600, (1,), generator=g))
        co = 4 * int(torch.randint(1, 200, (1,), generator=g))
        dens = [0.02, 0.1, 0.5][int(torch.randint(0, 3, (1,), generator=g))]
        out.append((m, k, co, dens))
    return out


@pytest.mark.parametrize("case", _random_linear_cases(20, 909))
@pytest.mark.parametrize("kernel", ["walk", "mfma", "mfma_bits"])
def test_linear_random_shapes(case, kernel):
    # Random (m, k, c_out): ragged row and column blocks, grids of every size
    # (the matrix-core kernel's XCD-local placement is a bijection for any
    # grid), walk workgroups of one to sixteen wavefronts.
    m, k, co, dens = case
    announce(f"linear random {kernel} {case}")
    x = spikes((m, k), dens, seed=m + 3 * k)
    w = _w(co, k, seed=co + m)
    b = torch.randn(co, generator=torch.Generator().manual_seed(k)) * 0.1
    y, kernels = _run(x.to(DEV), w.to(DEV), b.to(DEV), kernel=kernel)
    assert ("linear_flat" if kernel == "walk" else "linear_mfma") in kernels, kernels
    ok, err, _ = close(y, olin.linear_ref(x, w, b), **FP32_TOL)
    assert ok, f"max abs err {err}"
