"""Stage-2 sparse conv on the GPU vs the dense-conv oracle.

Tolerances: fp32 within 1e-4 abs + 1e-4 rel of
F.conv2d in float64; fp16/bf16 activations within 1e-2.  The oracle input is
the spike-masked x (elements with f16(|x|) <= f16(1e-6) are zero), which
equals x for spikes and ordinary values.
"""

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import conv as oconv
from sparseflow_amd import _lib
from sparseflow_amd.Kernels.conv2d import sparse_conv2d_forward
from sparseflow_amd.Ops.sparse_conv2d import SparseConv2d
from tests.gpu_helpers import DEV, announce, clustered_spikes, close, native_loaded, spikes

pytestmark = pytest.mark.gpu

FP32_TOL = dict(atol=1e-4, rtol=1e-4)


def _weights(c_out, c_in, k, seed=0, scale=None):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(c_out, c_in, k, k, generator=g)
    return w * (scale if scale is not None else (2.0 / (c_in * k * k)) ** 0.5)


CASES = [
    # (N, C_in, H, W, C_out, k, s)
    (32, 64, 32, 32, 64, 3, 1),
    (4, 64, 56, 56, 64, 3, 1),
    (4, 128, 28, 28, 128, 3, 1),
    (4, 64, 56, 56, 128, 3, 2),
    (4, 256, 14, 14, 256, 3, 1),
    (2, 512, 14, 14, 512, 3, 2),
    (4, 256, 28, 28, 64, 1, 1),
    (3, 3, 17, 13, 40, 3, 1),     # C_in < 32, C_out not a multiple of 64
    (2, 96, 9, 7, 200, 3, 2),     # ragged everything
    (2, 2048, 7, 7, 64, 1, 1),    # widest C_in
    (1, 16, 1, 1, 8, 3, 1),
]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("density", [0.0, 0.01, 0.2])
def test_conv_fp32_matches_dense(case, density):
    N, C, H, W, Co, k, s = case
    p = (k - 1) // 2
    announce(f"conv {case} p={density}")
    x = spikes((N, C, H, W), density, seed=N * 7 + C)
    w = _weights(Co, C, k, seed=C)
    b = torch.randn(Co, generator=torch.Generator().manual_seed(5)) * 0.1
    y, ms, meta = sparse_conv2d_forward(x.to(DEV), w.to(DEV), b.to(DEV), kernel_size=k, stride=s, padding=p,
                                        return_backend_meta=True)
    torch.cuda.synchronize()
    assert meta["backend"] == "sparse_hip"
    ref = oconv.sparse_conv2d_ref(x, w, b, s, p)
    ok, err, _ = close(y, ref, **FP32_TOL)
    assert ok, f"max abs err {err}"
    assert native_loaded()


@pytest.mark.parametrize("case", [(4, 64, 16, 16, 64, 3, 1), (2, 40, 11, 9, 130, 3, 2), (3, 256, 14, 14, 64, 1, 1)])
def test_conv_value_path_nonbinary(case):
    N, C, H, W, Co, k, s = case
    p = (k - 1) // 2
    g = torch.Generator().manual_seed(8)
    x = spikes((N, C, H, W), 0.1, seed=2) * torch.randn(N, C, H, W, generator=g)
    x[0, 0, 0, 0] = 3e-7       # below the activity threshold: dropped
    x[0, 1, 0, 0] = 1.2e-6     # above: kept
    w = _weights(Co, C, k, seed=3)
    announce(f"conv value path {case}")
    y = sparse_conv2d_forward(x.to(DEV), w.to(DEV), None, kernel_size=k, stride=s, padding=p)[0]
    ref = oconv.sparse_conv2d_ref(x, w, None, s, p)
    ok, err, _ = close(y, ref, **FP32_TOL)
    assert ok, f"max abs err {err}"


def test_conv_dense_input_matches_dense():
    # Fully dense non-binary input exercises entry-list batching (many
    # entries per pixel) and the value path everywhere.
    x = torch.randn(2, 512, 9, 9, generator=torch.Generator().manual_seed(1))
    w = _weights(96, 512, 3, seed=2)
    announce("conv dense 512")
    y = sparse_conv2d_forward(x.to(DEV), w.to(DEV), None, kernel_size=3, stride=1, padding=1)[0]
    ok, err, _ = close(y, oconv.conv2d_ref(x, w, None, 1, 1), **FP32_TOL)
    assert ok, f"max abs err {err}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("k,s", [(3, 1), (3, 2), (1, 1)])
def test_conv_half_activations(dtype, k, s):
    p = (k - 1) // 2
    x = spikes((4, 64, 20, 20), 0.05, seed=4)
    w = _weights(64, 64, k, seed=6)
    announce(f"conv {dtype} k{k}s{s}")
    y = sparse_conv2d_forward(x.to(DEV, dtype), w.to(DEV), None, kernel_size=k, stride=s, padding=p)[0]
    assert y.dtype == dtype
    ok, err, _ = close(y, oconv.conv2d_ref(x, w, None, s, p), atol=1e-2, rtol=1e-2)
    assert ok, f"max abs err {err}"
    y32 = sparse_conv2d_forward(x.to(DEV, dtype), w.to(DEV), None, kernel_size=k, stride=s, padding=p,
                                output_dtype=torch.float32)[0]
    assert y32.dtype == torch.float32
    ok, err, _ = close(y32, oconv.conv2d_ref(x, w, None, s, p), **FP32_TOL)
    assert ok, f"max abs err {err}"


def test_conv_deterministic_bitwise():
    x = spikes((8, 128, 28, 28), 0.02, seed=12).to(DEV)
    w = _weights(128, 128, 3, seed=13).to(DEV)
    announce("conv determinism")
    y1 = sparse_conv2d_forward(x, w, None, 3, 1, 1)[0]
    y2 = sparse_conv2d_forward(x, w, None, 3, 1, 1)[0]
    assert torch.equal(y1, y2)


def test_conv_golden_fixture():
    from tests.golden import load_golden

    g = load_golden("conv_golden.npz")
    for i in range(int(g["count"])):
        k, s, p = (int(v) for v in g[f"geom{i}"])
        x, w = torch.from_numpy(g[f"x{i}"]), torch.from_numpy(g[f"w{i}"])
        b = torch.from_numpy(g[f"b{i}"]) if g[f"b{i}"].size else None
        announce(f"golden conv {i}")
        y = sparse_conv2d_forward(x.to(DEV), w.to(DEV), None if b is None else b.to(DEV), k, s, p)[0]
        ok, err, _ = close(y, torch.from_numpy(g[f"y{i}"]), **FP32_TOL)
        assert ok, f"case {i}: max abs err {err}"


def _sampled_check(y, x_cpu, w_cpu, b_cpu, s, p, n_samples=256, seed=0):
    rng = np.random.default_rng(seed)
    N, Co, Ho, Wo = y.shape
    xn, wn = x_cpu.numpy(), w_cpu.numpy()
    bn = None if b_cpu is None else b_cpu.numpy()
    idx = [(int(rng.integers(N)), int(rng.integers(Co)), int(rng.integers(Ho)), int(rng.integers(Wo)))
           for _ in range(n_samples)]
    idx += [(0, 0, 0, 0), (N - 1, Co - 1, Ho - 1, Wo - 1)]
    yc = y.cpu()
    for (n, co, oh, ow) in idx:
        ref = oconv.conv2d_at(xn, wn, bn, s, p, n, co, oh, ow)
        got = float(yc[n, co, oh, ow])
        assert abs(got - ref) <= 1e-4 + 1e-4 * abs(ref), (n, co, oh, ow, got, ref)


@pytest.mark.parametrize("name,shape,co,k,s,gen", [
    ("resnet50_layer1_conv3x3", (512, 64, 56, 56), 64, 3, 1, "iid"),
    ("resnet50_layer2_conv3x3", (512, 128, 28, 28), 128, 3, 1, "iid"),
    ("resnet50_layer3_0_conv3x3_s2", (512, 256, 28, 28), 256, 3, 2, "iid"),
    ("config2_conv1x1", (512, 256, 56, 56), 64, 1, 1, "clustered"),
])
def test_full_size_sampled(name, shape, co, k, s, gen):
    """BASELINE full sizes: exact oracle values at sampled outputs, plus a
    size-independent identity (all-zero input gives the bias everywhere)."""
    p = (k - 1) // 2
    announce(f"full size {name}")
    x = spikes(shape, 0.01, seed=1) if gen == "iid" else clustered_spikes(shape, seed=1)
    w = _weights(co, shape[1], k, seed=2)
    b = torch.randn(co, generator=torch.Generator().manual_seed(3)) * 0.1
    xd = x.to(DEV)
    y = sparse_conv2d_forward(xd, w.to(DEV), b.to(DEV), k, s, p)[0]
    torch.cuda.synchronize()
    _sampled_check(y, x, w, b, s, p)
    del y
    z = sparse_conv2d_forward(torch.zeros(4, *shape[1:], device=DEV), w.to(DEV), b.to(DEV), k, s, p)[0]
    assert torch.equal(z, b.to(DEV).view(1, -1, 1, 1).expand_as(z))


def test_api_tuple_arity_and_metadata():
    x = spikes((4, 64, 56, 56), 0.01, seed=3).to(DEV)
    w = _weights(64, 64, 3, seed=4).to(DEV)
    announce("api arity")
    ag = torch.empty(4 * 7 * 4, dtype=torch.int32, device=DEV)
    tc = torch.empty_like(ag)
    out = sparse_conv2d_forward(x, w, None, 3, 1, 1, ag_mask_buf=ag, tile_class_buf=tc, return_ms=True,
                                return_avg_active_ratio=True, return_tile_stats=True, return_backend_meta=True)
    assert len(out) == 5
    y, ms, ratio, stats, meta = out
    assert ms > 0.0 and 0.0 <= ratio <= 1.0
    assert stats["total_tiles"] == 4 * 7 * 4
    assert meta["backend"] == "sparse_hip"
    from oracle import prescan as op

    ag_ref, tc_ref, _ = op.prescan_reference_geometry(x.cpu().numpy(), 3, 1, 1)
    np.testing.assert_array_equal(ag.cpu().numpy(), ag_ref)
    np.testing.assert_array_equal(tc.cpu().numpy(), tc_ref)
    # Unsupported patterns fall back to dense, as in the reference.
    w5 = _weights(8, 64, 5, seed=1).to(DEV)
    y5, _, meta5 = sparse_conv2d_forward(x, w5, None, 5, 1, 2, return_backend_meta=True)
    assert meta5["reason"] == "unsupported_pattern"
    w1 = _weights(8, 64, 1, seed=1).to(DEV)
    _, _, meta_s2 = sparse_conv2d_forward(x, w1, None, 1, 2, 0, return_backend_meta=True)
    assert meta_s2["reason"] == "split_1x1s2_downsample"
    # All-zero input: stats report zero tiles.
    *_, meta0 = sparse_conv2d_forward(torch.zeros_like(x), w, None, 3, 1, 1, return_tile_stats=True,
                                      return_backend_meta=True)
    assert meta0["backend"] == "zero_tiles_only"


@pytest.mark.parametrize("k,s", [(3, 1), (3, 2), (1, 1)])
def test_module_from_dense_4d_and_5d(k, s):
    p = (k - 1) // 2
    conv = nn.Conv2d(64, 96, k, s, p, bias=True).to(DEV)
    sp = SparseConv2d.from_dense(conv, block_size=8)
    x5 = spikes((4, 3, 64, 24, 24), 0.03, seed=k * 10 + s).to(DEV)
    announce(f"module k{k}s{s}")
    with torch.no_grad():
        y5 = sp(x5)
        ref5 = oconv.conv2d_ref(x5.reshape(12, 64, 24, 24), conv.weight, conv.bias, s, p)
    assert y5.shape == (4, 3, 96, *ref5.shape[-2:])
    ok, err, _ = close(y5.reshape(ref5.shape), ref5, **FP32_TOL)
    assert ok, f"max abs err {err}"
    with torch.no_grad():
        y4 = sp(x5[1])
    assert torch.equal(y4, y5[1])
    sp.collect_diag = True
    sp.return_ms = True
    with torch.no_grad():
        sp(x5)
    d = sp._last_diag
    assert d["backend"] == "sparse_hip" and d["block_size"] == 8 and sp._last_sparse_ms > 0
    # Weight updates invalidate the cached tap-major weights.
    with torch.no_grad():
        sp.weight.mul_(2.0)
        y_scaled = sp(x5)
        conv.weight.mul_(2.0)
        ref_scaled = oconv.conv2d_ref(x5.reshape(12, 64, 24, 24), conv.weight, conv.bias, s, p)
    ok, err, _ = close(y_scaled.reshape(ref_scaled.shape), ref_scaled, **FP32_TOL)
    assert ok, f"max abs err {err}"


def test_module_fp16_weights_config2_style():
    conv = nn.Conv2d(256, 64, 1, bias=False).half().to(DEV)
    sp = SparseConv2d.from_dense(conv)
    assert sp.weight.dtype == torch.float32
    x = clustered_spikes((2, 4, 256, 28, 28), seed=4).to(DEV)
    announce("module fp16 weights")
    with torch.no_grad():
        y = sp(x)
    ref = oconv.conv2d_ref(x.reshape(8, 256, 28, 28), conv.weight.float(), None, 1, 0)
    ok, err, _ = close(y.reshape(ref.shape), ref, **FP32_TOL)
    assert ok, f"max abs err {err}"


def test_missing_library_fails_loudly(monkeypatch):
    from sparseflow_amd import _lib as L

    monkeypatch.setattr(L, "_lib", None)
    monkeypatch.setattr(L, "LIB_PATH", L.LIB_PATH.with_name("does_not_exist.so"))
    x = spikes((1, 8, 8, 8), 0.1).to(DEV)
    w = _weights(8, 8, 3).to(DEV)
    with pytest.raises(L.SparseFlowLibError):
        sparse_conv2d_forward(x, w, None, 3, 1, 1)
