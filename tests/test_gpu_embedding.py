"""The owner's token-embedding gradient on the GPU, against torch's own aten.embedding_dense_backward on the same
device (the routine the reference calls, yoco/models/decoder/layer_graphs.py:92, ce_reduce.py:230) and against the
oracle.  aten takes its sort-based path for more than 3072 indices and another kernel for fewer; this build follows
the order of each (bit-exact)."""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def zipf_ids(rng, R, V, a=1.2):
    ids = rng.zipf(a, R) - 1
    return np.where(ids < V, ids, rng.integers(0, V, R)).astype(np.int64)


def bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize('padding_idx', [-1, 1])
@pytest.mark.parametrize('D', [3072, 200])
def test_matches_aten_sort_path(pkg, dev, padding_idx, D):
    from faster_yoco_amd import embedding
    rng = np.random.default_rng(D + padding_idx)
    R, V = 8 * 2048, 100288
    ids = torch.from_numpy(zipf_ids(rng, R, V)).to(dev)
    assert int((ids == 0).sum()) > 100                       # long runs: many partials of 10
    g = (torch.randn(R, D, device=dev) * 1e-2).to(torch.bfloat16)
    ref = torch.ops.aten.embedding_dense_backward(g, ids, V, padding_idx, False)
    got = embedding.embedding_dense_backward(g, ids, V, padding_idx)
    torch.cuda.synchronize()
    assert np.array_equal(bits(got), bits(ref))
    # the reference's two 1/world placements
    ref2 = torch.ops.aten.embedding_dense_backward(g, ids, V, padding_idx, False).mul_(1.0 / 8)
    got2 = embedding.owner_embedding_grad(g, ids, V, padding_idx, 8)
    ref3 = torch.ops.aten.embedding_dense_backward(g.clone().mul_(1.0 / 8), ids, V, padding_idx, False)
    got3 = embedding.ce_owner_embedding_grad(g, ids, V, padding_idx, 8)
    torch.cuda.synchronize()
    assert np.array_equal(bits(got2), bits(ref2)) and np.array_equal(bits(got3), bits(ref3))


@pytest.mark.parametrize('R', [65536, 1_500_000])
def test_matches_aten_at_larger_row_counts(pkg, dev, R):
    """More rows than the recipe's 16,384: the sort runs rocPRIM's other algorithms (merge sort up to 1M items,
    onesweep above); still bit-exact against aten."""
    from faster_yoco_amd import embedding
    rng = np.random.default_rng(R)
    V, D = 100288, 64
    ids = torch.from_numpy(zipf_ids(rng, R, V)).to(dev)
    g = (torch.randn(R, D, device=dev) * 1e-2).to(torch.bfloat16)
    ref = torch.ops.aten.embedding_dense_backward(g, ids, V, -1, False)
    got = embedding.embedding_dense_backward(g, ids, V, -1)
    torch.cuda.synchronize()
    assert np.array_equal(bits(got), bits(ref))


@pytest.mark.parametrize('D', [3072, 40, 13])
def test_heavy_ids_at_the_run_boundaries(pkg, dev, D):
    """Ids with 20 occurrences (the rows kernel's most), 21 (the heavy passes' fewest), 30, 31, 320 (the most one
    wave chains: 32 runs), 321 and 9,878; 400 ids
    with exactly 21 each, which fill every run slot the workspace holds (R / 7); one id taking every row.  Against
    aten's sort path (more than 3072 rows in every case), on the vector path with several and with one partial
    column group, and on the element path."""
    from faster_yoco_amd import embedding
    rng = np.random.default_rng(D)
    V = 5000
    mix = np.concatenate([np.full(c, t) for t, c in ((7, 20), (8, 21), (9, 30), (10, 31), (11, 9878), (12, 1),
                                                     (13, 320), (14, 321))] + [rng.integers(15, V, 3000)])
    cases = [rng.permutation(mix), rng.permutation(np.repeat(np.arange(100, 500), 21)), np.full(16384, 4)]
    for ids in cases:
        ids = torch.from_numpy(ids.astype(np.int64)).to(dev)
        R = ids.numel()
        g = (torch.randn(R, D, device=dev) * 1e-2).to(torch.bfloat16)
        for pad in (-1, 8):
            ref = torch.ops.aten.embedding_dense_backward(g, ids, V, pad, False)
            got = embedding.embedding_dense_backward(g, ids, V, pad)
            torch.cuda.synchronize()
            assert np.array_equal(bits(got), bits(ref)), (R, pad)


@pytest.mark.parametrize('D', [3072, 40, 13])
def test_matches_aten_at_3072_rows_or_fewer(pkg, dev, D):
    """At most 3072 rows: aten's kernel for few indices, whose order (chunks of 16 indices, each chunk's sum rounded to
    bf16 and added to the bf16 row) this build follows there.  Bit-exact against torch's aten for 1 row, for chunk
    boundaries (15, 16, 17 rows), and up to 3072 rows with heavy repeats, padding and both 1/world placements."""
    from faster_yoco_amd import embedding
    rng = np.random.default_rng(100 + D)
    for R, V in ((1, 5), (15, 3), (16, 3), (17, 3), (1000, 7), (2048, 300), (3072, 40), (3072, 100288)):
        ids = torch.from_numpy(rng.integers(0, V, R).astype(np.int64)).to(dev)
        g = (torch.randn(R, D, device=dev) * 1e-2).to(torch.bfloat16)
        for pad in (-1, 2):
            ref = torch.ops.aten.embedding_dense_backward(g, ids, V, pad, False)
            got = embedding.embedding_dense_backward(g, ids, V, pad)
            torch.cuda.synchronize()
            assert np.array_equal(bits(got), bits(ref)), (R, V, pad)
        ref2 = torch.ops.aten.embedding_dense_backward(g, ids, V, -1, False).mul_(1.0 / 8)
        ref3 = torch.ops.aten.embedding_dense_backward(g.clone().mul_(1.0 / 8), ids, V, -1, False)
        got2 = embedding.owner_embedding_grad(g, ids, V, -1, 8)
        got3 = embedding.ce_owner_embedding_grad(g, ids, V, -1, 8)
        torch.cuda.synchronize()
        assert np.array_equal(bits(got2), bits(ref2)) and np.array_equal(bits(got3), bits(ref3)), R


def test_matches_oracle_and_edge_cases(pkg, dev):
    from faster_yoco_amd import embedding
    rng = np.random.default_rng(3)
    R, V, D = 4000, 300, 13                                   # D % 8 != 0: the element path
    ids = zipf_ids(rng, R, V, 1.5)
    ids[:4] = [-5, V, V + 7, 2 ** 40]                         # outside [0, V): contribute nothing
    g16 = oracle.bf16_rne((rng.standard_normal((R, D)) * 1e-2).astype(np.float32))
    for pad, scale, first in ((-1, None, False), (3, 0.125, False), (0, 0.125, True)):
        exp = oracle.embedding_backward(ids, g16, V, padding_idx=pad, scale=scale, scale_first=first)
        gt = torch.from_numpy(g16.view(np.int16)).to(dev).view(torch.bfloat16)
        got = embedding.embedding_dense_backward(gt, torch.from_numpy(ids).to(dev), V, pad, scale=scale,
                                                 scale_first=first)
        torch.cuda.synchronize()
        assert np.array_equal(bits(got), exp)
    # no rows at all: a zero table; a preexisting out buffer is fully overwritten
    out = torch.full((V, 16), 7.0, dtype=torch.bfloat16, device=dev)
    embedding.embedding_dense_backward(torch.zeros(0, 16, dtype=torch.bfloat16, device=dev),
                                       torch.zeros(0, dtype=torch.int64, device=dev), V, -1, out=out)
    torch.cuda.synchronize()
    assert not out.float().abs().sum().item()
    with pytest.raises(RuntimeError, match='scale_grad_by_freq'):
        embedding.embedding_dense_backward(gt, torch.from_numpy(ids).to(dev), V, -1, True)


def test_aten_few_indices_order_known_answer(pkg, dev):
    """Guard of the bit-exact claim for at most 3072 rows, whose order follows torch's own ROCm aten kernel (chunks
    of 16 indices, each chunk's fp32 sum rounded to bf16 before it is added to the row).  On one id, rows 1.0, 2^-9,
    fourteen zeros, 2^-8: chunks of 16 give 0x3F80; one chunk of 32, or the sort path, 0x3F81.  If a torch build
    walks the indices otherwise, this fails here, loudly, instead of the bf16 copies drifting in their last bit."""
    from faster_yoco_amd import embedding
    vals = [1.0, 2.0 ** -9] + [0.0] * 14 + [2.0 ** -8]
    g = torch.tensor(vals, dtype=torch.float32).reshape(-1, 1).to(torch.bfloat16).to(dev)
    ids = torch.zeros(len(vals), dtype=torch.int64, device=dev)
    aten = torch.ops.aten.embedding_dense_backward(g, ids, 1, -1, False)
    ours = embedding.embedding_dense_backward(g, ids, 1, -1)
    torch.cuda.synchronize()
    assert int(aten.view(torch.int16).item()) & 0xFFFF == 0x3F80, 'torch\'s few-indices order changed'
    assert int(ours.view(torch.int16).item()) & 0xFFFF == 0x3F80
