"""Debug mode (ACTKV_DEBUG=1): every compaction launch's per-request report {kept, moved,
dropped, remaining blocks} is read back and must equal the host's counts, and the plan's
sources and destinations must be distinct and disjoint (reference compaction.py:3-13, :61).
Normal evictions pass it; the state still matches the oracle bit for bit."""
import math

import numpy as np
import pytest
import torch

from actkv.paged import PagedKVCache
from oracle import reference as ref

pytestmark = pytest.mark.gpu


def _cache(lens, layers, seed, dtype=torch.bfloat16, bs=16, hkv=4, d=64):
    g = torch.Generator().manual_seed(seed)
    nb = sum(math.ceil(s / bs) for s in lens) + 8
    cache = PagedKVCache(nb, bs, hkv, d, n_layers=layers, dtype=dtype, device="cuda")
    cache.free = torch.randperm(nb, generator=g).tolist()
    model = ref.PagedCacheModel(nb, bs, hkv, d, layers)
    model.free = list(cache.free)
    for r, s in enumerate(lens):
        k = torch.randn(layers, s, hkv, d, generator=g).to(dtype)
        v = torch.randn(layers, s, hkv, d, generator=g).to(dtype)
        cache.append(r, k.cuda(), v.cuda())
        model.append(r, k.view(torch.int16).numpy().view(np.uint16), v.view(torch.int16).numpy().view(np.uint16))
    return cache, model, g


def test_debug_mode_batched_evictions_match_the_oracle(monkeypatch):
    monkeypatch.setenv("ACTKV_DEBUG", "1")
    lens = [1000, 37, 4097, 300]
    cache, model, g = _cache(lens, 2, 11)
    for rnd, budgets in enumerate(([200, 10, 900, 400], [50, 5, 300, 20])):
        scores = [torch.rand(2, 4, cache.seq_used[r], generator=g) for r in range(4)]
        perms = cache.evict_batch([0, 1, 2, 3], [s.cuda() for s in scores], budgets, protected=[4, 0, 8, 2])
        for r in range(4):
            perm_o = model.evict(r, scores[r], budgets[r], protected=[4, 0, 8, 2][r])
            assert np.array_equal(perms[r].cpu().numpy(), perm_o), (rnd, r)
        kv = cache.kv.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(kv, model.kv)
        assert cache.free == model.free and cache.tables == model.tables and cache.seq_used == model.seq_used
        for r in range(4):
            assert np.array_equal(cache.pinned[r].cpu().numpy(), model.pinned[r])


def test_debug_mode_compact_with_a_caller_mask(monkeypatch):
    monkeypatch.setenv("ACTKV_DEBUG", "1")
    cache, model, g = _cache([777], 1, 12, dtype=torch.float16)
    keep = torch.rand(777, generator=g) < 0.3
    perm = cache.compact(0, keep.cuda())
    perm_o = model.compact(0, keep.numpy())
    assert np.array_equal(perm.cpu().numpy(), perm_o)
    assert np.array_equal(cache.kv.cpu().view(torch.int16).numpy().view(np.uint16), model.kv)
    assert cache.free == model.free and cache.tables == model.tables


def test_evict_after_a_compact_refuses_stale_pins():
    """compact() does not remap the stored pins (paged.py:125-139), so a following evict()
    finds more pins than tokens and raises, as the reference's pad of negative length does."""
    cache, _, g = _cache([500], 1, 13)
    cache.evict(0, torch.rand(500, generator=g).cuda(), budget=600, protected=4)   # within budget: pins stored
    assert cache.pinned[0].numel() == 500
    cache.compact(0, (torch.rand(500, generator=g) < 0.5).cuda())
    with pytest.raises(RuntimeError, match="pinned"):
        cache.evict(0, torch.rand(cache.seq_used[0], generator=g).cuda(), budget=10)
