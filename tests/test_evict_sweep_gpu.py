"""Eviction (keep mask + compaction, paged.py:23-46 and :125-157) over a seeded random sweep of
shapes, against the oracle's PagedCacheModel, bit-exact.

Each case draws 1-4 requests of 1-3000 tokens, 1-3 layers, Hkv 1/2/8, head_dim 16/32/128,
block 8/16/32, a float32, bf16 or fp16 cache, and a shuffled free stack; then two rounds:
  1. a first eviction per request (budget 0..S, a protected prefix 0..40);
  2. appends of 0-200 tokens, then a repeated eviction (the pins follow their tokens), as one
     evict_batch call or request by request.
After every step: the permutations and pinned masks, the whole K/V tensor's bits, the free
stack, the block tables and seq_used equal the model's.  Scores are continuous random
numbers; ties at the k-th score take the lowest index on both sides (tie_rule "lowest").
"""
import math
import random

import numpy as np
import pytest
import torch

from actkv.paged import PagedKVCache
from oracle import reference as ref

pytestmark = pytest.mark.gpu


def _bits(t):
    t = t.detach().cpu().contiguous()
    return t.view({4: torch.int32, 2: torch.int16, 1: torch.uint8}[t.element_size()]).numpy()


def _same_state(cache, model):
    assert np.array_equal(_bits(cache.kv), model.kv), "KV bytes differ"
    assert cache.free == model.free
    assert {r: list(t) for r, t in cache.tables.items()} == model.tables
    assert cache.seq_used == model.seq_used


@pytest.mark.parametrize("seed", range(48))
def test_random_evictions_match_the_model(seed):
    rnd = random.Random(2000 + seed)
    lens = [rnd.choice([rnd.randint(1, 100), rnd.randint(100, 3000)]) for _ in range(rnd.randint(1, 4))]
    layers, hkv = rnd.randint(1, 3), rnd.choice([1, 2, 8])
    d, bs = rnd.choice([16, 32, 128]), rnd.choice([8, 16, 32])
    dtype = rnd.choice([torch.float32, torch.bfloat16, torch.float16])
    extra = [rnd.randint(0, 200) for _ in lens]
    batched = rnd.random() < 0.5
    print(f"case {seed}: lens {lens} extra {extra} L {layers} Hkv {hkv} D {d} bs {bs} {dtype} "
          f"batched {batched}", flush=True)
    g = torch.Generator().manual_seed(seed)
    nb = sum(math.ceil((n + e) / bs) for n, e in zip(lens, extra)) + 6
    cache = PagedKVCache(nb, bs, hkv, d, n_layers=layers, dtype=dtype, device="cuda")
    cache.free = torch.randperm(nb, generator=g).tolist()
    model = ref.PagedCacheModel(nb, bs, hkv, d, layers, np_dtype=_bits(cache.kv[:1, :1, :1]).dtype)
    model.free = list(cache.free)

    def append(r, n):
        k = torch.randn(layers, n, hkv, d, generator=g).to(dtype)
        v = torch.randn(layers, n, hkv, d, generator=g).to(dtype)
        cache.append(r, k.cuda(), v.cuda())
        model.append(r, _bits(k), _bits(v))

    def evict_one(r, budget, protected):
        s = torch.rand(layers, hkv, cache.seq_used[r], generator=g)
        perm = cache.evict(r, s.cuda(), budget=budget, protected=protected)
        want = model.evict(r, s, budget=budget, protected=protected, tie_rule="lowest")
        assert np.array_equal(perm.cpu().numpy(), want), r
        assert np.array_equal(cache.pinned[r].cpu().numpy(), model.pinned[r]), r

    for r, n in enumerate(lens):
        append(r, n)
    _same_state(cache, model)
    for r, n in enumerate(lens):
        evict_one(r, rnd.randint(0, n), rnd.randint(0, min(n, 40)))
    _same_state(cache, model)
    for r, e in enumerate(extra):
        if e:
            append(r, e)
    _same_state(cache, model)
    budgets = [rnd.randint(0, cache.seq_used[r]) for r in range(len(lens))]
    if batched:
        scores = [torch.rand(layers, hkv, cache.seq_used[r], generator=g) for r in range(len(lens))]
        perms = cache.evict_batch(list(range(len(lens))), [s.cuda() for s in scores], budgets, [0] * len(lens))
        for r in range(len(lens)):
            want = model.evict(r, scores[r], budget=budgets[r], protected=0, tie_rule="lowest")
            assert np.array_equal(perms[r].cpu().numpy(), want), r
            assert np.array_equal(cache.pinned[r].cpu().numpy(), model.pinned[r]), r
    else:
        for r in range(len(lens)):
            evict_one(r, budgets[r], 0)
    _same_state(cache, model)
