"""Pins the sparse Linear / batched-matmul oracle (oracle/linear.py) and the
host-side metadata derivation, on the CPU.

  row_bitmap           vs a per-element loop over prescan.active_elements
  linear_ref/bmm_ref   vs brute-force triple loops in float64, and the
                       identity that masked-out elements contribute nothing
  tile_group_metadata  vs the reference's three-pass description evaluated
                       literally (representative channel, zero-candidate
                       refine from channel 1, exact refine)
  Kernels.linear.group_metadata (product, used for statistics) vs the oracle
"""

import numpy as np
import pytest
import torch

from oracle import linear as olin
from oracle.prescan import active_elements, choose_group_size
from sparseflow_amd.Kernels.linear import _select_linear_block_m, group_metadata


def _spikes(shape, p, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.rand(shape, generator=g) < p).float()


@pytest.mark.parametrize("m,k", [(1, 1), (3, 31), (5, 33), (7, 64), (4, 100), (6, 130), (2, 384)])
def test_row_bitmap_matches_element_loop(m, k):
    x = _spikes((m, k), 0.3, m * 100 + k).numpy()
    x[0, 0] = 3e-7   # below the threshold: inactive
    x[-1, -1] = -2.0
    bits = olin.row_bitmap(x, 1e-6)
    act = active_elements(x, 1e-6)
    words = olin.linear_words_per_row(k)
    assert bits.shape == (m, words)
    assert words in (1, 2) or words % 4 == 0
    for r in range(m):
        for j in range(words * 32):
            want = bool(act[r, j]) if j < k else False
            assert bool((int(bits[r, j // 32]) >> (j % 32)) & 1) == want


def test_linear_ref_brute_force():
    g = torch.Generator().manual_seed(1)
    x = _spikes((5, 7), 0.5, 2) * torch.tensor([1.0, 2.0, -0.5, 1.0, 1.0, 4e-7, 1.0])
    w = torch.randn(6, 7, generator=g)
    b = torch.randn(6, generator=g)
    y = olin.linear_ref(x, w, b)
    xa, wa, ba = x.double().numpy(), w.double().numpy(), b.double().numpy()
    for r in range(5):
        for o in range(6):
            acc = ba[o]
            for c in range(7):
                if abs(xa[r, c]) > 1e-6:   # 4e-7 is masked out, the rest kept
                    acc += xa[r, c] * wa[o, c]
            assert abs(float(y[r, o]) - acc) < 1e-12


def test_bmm_ref_brute_force_and_mask():
    g = torch.Generator().manual_seed(3)
    a = _spikes((2, 3, 5), 0.5, 4)
    a[0, 0, 0] = 1e-8
    b = torch.randn(2, 5, 4, generator=g)
    c = olin.bmm_ref(a, b)
    an, bn = a.double().numpy(), b.double().numpy()
    an_masked = np.where(np.abs(an) > 1e-6, an, 0.0)
    for bt in range(2):
        assert np.allclose(c[bt].numpy(), an_masked[bt] @ bn[bt], atol=1e-12)
    # Permuting the batch permutes the result.
    perm = torch.tensor([1, 0])
    assert torch.equal(olin.bmm_ref(a[perm], b[perm]), c[perm])


def _three_pass(active, block_m, gs):
    """The reference's linear metadata passes, evaluated literally."""
    rows, cols = active.shape
    ng = -(-cols // gs)
    all_ones = (1 << ng) - 1
    nt = -(-rows // block_m)
    masks, classes = [], []
    for t in range(nt):
        blk = active[t * block_m:(t + 1) * block_m]
        rough = 0
        for g in range(ng):
            if g * gs < cols and blk[:, g * gs].any():
                rough |= 1 << g
        if rough == all_ones:
            masks.append(all_ones)
            classes.append(2)
            continue
        mask = 0
        if rough == 0:  # zero candidate: channels 1.. of each group
            for g in range(ng):
                if blk[:, g * gs + 1:min((g + 1) * gs, cols)].any():
                    mask |= 1 << g
        else:           # uncertain: exact
            for g in range(ng):
                if blk[:, g * gs:min((g + 1) * gs, cols)].any():
                    mask |= 1 << g
        masks.append(mask)
        classes.append(0 if mask == 0 else (2 if mask == all_ones else 1))
    return np.array(masks, dtype=np.int64), np.array(classes, dtype=np.int32)


@pytest.mark.parametrize("rows,cols,p", [(70, 40, 0.02), (300, 384, 0.001), (33, 16, 0.5), (129, 1000, 0.0005)])
def test_group_metadata_oracle_and_product(rows, cols, p):
    act = (_spikes((rows, cols), p, rows + cols) > 0).numpy()
    bm = _select_linear_block_m(rows)
    gs = choose_group_size(cols)
    m_o, c_o = olin.tile_group_metadata(act, bm, gs)
    m3, c3 = _three_pass(act, bm, gs)
    m3 = np.where(m3 >= (1 << 31), m3 - (1 << 32), m3).astype(np.int32)
    assert np.array_equal(m_o, m3) and np.array_equal(c_o, c3)
    m_p, c_p, ng = group_metadata(torch.from_numpy(act), bm, gs)
    assert ng == -(-cols // gs)
    assert np.array_equal(m_p.numpy(), m_o) and np.array_equal(c_p.numpy(), c_o)


def test_nonbinary_chunks():
    x = _spikes((40, 8), 0.3, 9).numpy()
    x[17, 2] = 2.0
    nb = olin.row_chunk_nonbinary(x)
    assert nb.tolist() == [False, True, False]
