"""Sparse batched matmul and attention stages on the GPU (sf_bmm_sparse via
Kernels.bmm / Kernels.attention / SparseAttention).

Bar: fp32 within 1e-4 abs + 1e-4 rel of float64 torch.bmm on the activity-
masked A; fp16/bf16 within 1e-2; K^T read through strides equals the
contiguous copy bit for bit."""

import pytest
import torch

from oracle import linear as olin
from sparseflow_amd import _lib
from sparseflow_amd.Kernels.attention import sparse_attn_v_forward, sparse_qk_forward
from sparseflow_amd.Kernels.bmm import sparse_bmm_forward
from sparseflow_amd.Ops import SparseAttention, SparseBMM, SparseMatmul
from tests.gpu_helpers import DEV, announce, close, native_loaded, spikes

pytestmark = pytest.mark.gpu

FP32_TOL = dict(atol=1e-4, rtol=1e-4)


def _run(a, b, **kw):
    torch.cuda.synchronize()
    _lib.timing_reset()
    _lib.timing_enable(True)
    try:
        c = sparse_bmm_forward(a, b, **kw)[0]
        torch.cuda.synchronize()
        stats = _lib.timing_collect()
    finally:
        _lib.timing_enable(False)
    return c, {k: n for k, (n, _) in stats.items() if n > 0}


CASES = [  # (batches, m, k, n)
    (1, 1, 1, 1), (3, 5, 7, 9), (48, 196, 32, 196), (48, 196, 196, 32), (4, 64, 252, 64), (2, 300, 64, 300),
    (5, 17, 130, 70), (2, 8, 40, 513),
    # More batches than resident workgroups: each workgroup takes several in
    # turn, and a wavefront's next tile is often in its next batch (m = 80:
    # five row tiles over four wavefronts; m = 20: two wavefronts idle).
    (2000, 80, 40, 24), (1500, 20, 32, 16),
    # Widest padded B rows in LDS (k 33..64 with n = 256: 96 KB).
    (3, 40, 64, 256),
]


def _expected_kernel(kernel, k, n):
    mfma = kernel != "walk" and _lib.bmm_mfma_supported(k, n)
    return "bmm_mfma" if mfma else "bmm_sparse"


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("density", [0.0, 0.1, 0.6])
@pytest.mark.parametrize("kernel", ["walk", "mfma"])
def test_bmm_fp32_matches_dense(case, density, kernel):
    bt, m, k, n = case
    announce(f"bmm {kernel} {case} p={density}")
    a = spikes((bt, m, k), density, seed=m + k)
    b = torch.randn(bt, k, n, generator=torch.Generator().manual_seed(n))
    c, kernels = _run(a.to(DEV), b.to(DEV), kernel=kernel)
    assert set(kernels) == {_expected_kernel(kernel, k, n)}, kernels
    ok, err, _ = close(c, olin.bmm_ref(a, b), **FP32_TOL)
    assert ok, f"max abs err {err}"
    assert native_loaded()


@pytest.mark.parametrize("kernel", ["walk", "mfma"])
def test_bmm_strided_b_equals_contiguous(kernel):
    a = spikes((24, 196, 32), 0.1, seed=1).to(DEV)
    k = spikes((24, 196, 32), 0.1, seed=2).to(DEV)
    announce(f"bmm strided K^T {kernel}")
    c1, _ = _run(a, k.transpose(1, 2), kernel=kernel)
    c2, _ = _run(a, k.transpose(1, 2).contiguous(), kernel=kernel)
    assert torch.equal(c1, c2)
    ok, err, _ = close(c1, olin.bmm_ref(a.cpu(), k.cpu().transpose(1, 2)), **FP32_TOL)
    assert ok, f"max abs err {err}"


@pytest.mark.parametrize("kernel", ["walk", "mfma"])
def test_bmm_general_strides_b(kernel):
    # B with neither axis contiguous (every other column of a wider tensor).
    a = spikes((6, 50, 70), 0.2, seed=8).to(DEV)
    wide = torch.randn(6, 70, 66, generator=torch.Generator().manual_seed(9)).to(DEV)
    b = wide[:, :, ::2]
    announce(f"bmm strided B {kernel}")
    c1, _ = _run(a, b, kernel=kernel)
    c2, _ = _run(a, b.contiguous(), kernel=kernel)
    assert torch.equal(c1, c2)
    ok, err, _ = close(c1, olin.bmm_ref(a.cpu(), b.cpu()), **FP32_TOL)
    assert ok, f"max abs err {err}"


@pytest.mark.parametrize("kernel", ["walk", "mfma"])
def test_bmm_value_a_and_half(kernel):
    g = torch.Generator().manual_seed(3)
    a = spikes((12, 196, 196), 0.3, seed=4) * torch.randint(1, 5, (12, 196, 196), generator=g).float() * 0.17
    b = spikes((12, 196, 32), 0.1, seed=5)
    announce(f"bmm attn @ v {kernel}")
    c, kernels = _run(a.to(DEV), b.to(DEV), kernel=kernel)
    assert set(kernels) == {_expected_kernel(kernel, 196, 32)}
    ok, err, _ = close(c, olin.bmm_ref(a, b), **FP32_TOL)
    assert ok, f"max abs err {err}"
    # Full fp32 mantissas in both operands: the hi + lo split keeps ~16 bits.
    b2 = torch.randn(12, 196, 32, generator=g)
    c2, _ = _run(a.to(DEV), b2.to(DEV), kernel=kernel)
    ok, err, _ = close(c2, olin.bmm_ref(a, b2), **FP32_TOL)
    assert ok, f"max abs err {err}"
    for dt in (torch.float16, torch.bfloat16):
        c, _ = _run(a.to(DEV, dt), b.to(DEV, dt), kernel=kernel)
        assert c.dtype == dt
        ok, err, _ = close(c, olin.bmm_ref(a.to(dt).float(), b.to(dt).float()), atol=1e-2, rtol=1e-2)
        assert ok, f"{dt}: max abs err {err}"


def test_bmm_large_k_falls_back():
    a = spikes((2, 8, 300), 0.1, seed=6)
    b = torch.randn(2, 300, 16, generator=torch.Generator().manual_seed(7))
    c, kernels = _run(a.to(DEV), b.to(DEV), return_tile_stats=True)
    assert not kernels
    ok, err, _ = close(c, olin.bmm_ref(a, b), **FP32_TOL)
    assert ok


def test_attention_stages_and_modules():
    T, N, H, S, D = 2, 3, 4, 50, 32
    q = spikes((T * N, H, S, D), 0.1, seed=8)
    k = spikes((T * N, H, S, D), 0.1, seed=9)
    v = spikes((T * N, H, S, D), 0.1, seed=10)
    announce("attention qk / av")
    attn, _ = sparse_qk_forward(q.to(DEV), k.to(DEV))
    ref_attn = torch.matmul(q.double(), k.double().transpose(-2, -1)) * D ** -0.5
    ok, err, _ = close(attn, ref_attn, **FP32_TOL)
    assert ok, f"qk err {err}"
    out, _ = sparse_attn_v_forward(attn, v.to(DEV))
    ok, err, _ = close(out, torch.matmul(ref_attn, v.double()), **FP32_TOL)
    assert ok, f"av err {err}"
    sa = SparseAttention(H, D)
    ok, _, _ = close(sa.av(sa.qk(q.to(DEV), k.to(DEV)), v.to(DEV)), torch.matmul(ref_attn, v.double()), **FP32_TOL)
    assert ok
    bm = SparseBMM()
    bm.collect_diag = True
    c = bm(q.reshape(-1, S, D).to(DEV), v.reshape(-1, S, D).transpose(1, 2).contiguous().to(DEV))
    assert c.shape == (T * N * H, S, S) and "total_tile_count" in bm._last_diag
    mm = SparseMatmul()
    a2 = spikes((70, 40), 0.2, seed=11)
    b2 = torch.randn(40, 24, generator=torch.Generator().manual_seed(12))
    ok, err, _ = close(mm(a2.to(DEV), b2.to(DEV)), olin.linear_ref(a2, b2.t(), None), **FP32_TOL)
    assert ok, f"matmul err {err}"
    b3 = torch.randn(40, 22, generator=torch.Generator().manual_seed(13))  # n % 4 != 0: batched path
    ok, err, _ = close(mm(a2.to(DEV), b3.to(DEV)), olin.linear_ref(a2, b3.t(), None), **FP32_TOL)
    assert ok, f"matmul (bmm path) err {err}"


@pytest.mark.parametrize("shape", [(8, 12, 196, 32), (4, 3, 64, 64), (6, 8, 50, 16), (2, 2, 300, 32)])
@pytest.mark.parametrize("p", [0.0, 0.1, 0.5])
def test_fused_spike_attention(shape, p):
    from sparseflow_amd.Kernels.attention import sparse_spike_attention_forward

    B, H, S, D = shape
    q, k, v = (spikes(shape, p, seed=s) for s in (20, 21, 22))
    q[0, 0, 0, :4] = torch.tensor([2.0, -0.5, 3e-7, 1.0])   # values and a sub-threshold element
    announce(f"spike attention {shape} p={p}")
    ref = torch.matmul(torch.matmul(olin.masked(q, 1e-6).double(), k.double().transpose(-2, -1)) * D ** -0.5,
                       v.double())
    _lib.timing_reset()
    _lib.timing_enable(True)
    y = sparse_spike_attention_forward(q.to(DEV), k.to(DEV), v.to(DEV))
    torch.cuda.synchronize()
    stats = _lib.timing_collect()
    _lib.timing_enable(False)
    assert stats["spike_attention"][0] == 1
    ok, err, _ = close(y, ref, **FP32_TOL)
    assert ok, f"max abs err {err}"
    # Token-major views give the same numbers.
    qt, kt, vt = (t.transpose(1, 2).contiguous().to(DEV) for t in (q, k, v))
    yt = sparse_spike_attention_forward(qt, kt, vt, token_major=True)
    assert torch.equal(yt.transpose(1, 2).cpu(), y.cpu())


def test_fused_spike_attention_unsupported_shapes():
    from sparseflow_amd.Kernels.attention import sparse_spike_attention_forward

    q = spikes((2, 2, 20, 48), 0.1, seed=23).to(DEV)
    assert sparse_spike_attention_forward(q, q, q) is None          # head_dim 48
    q = spikes((1, 1, 700, 64), 0.1, seed=24).to(DEV)
    assert sparse_spike_attention_forward(q, q, q) is None          # k, v exceed LDS
    assert not _lib.spike_attention_supported(700, 64) and _lib.spike_attention_supported(196, 32)
