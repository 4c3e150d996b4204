"""Paged attention with the LSE by-product over a seeded random sweep of shapes, against the
oracle's float64 restatement of lse_attn.py:42-60.

Each case draws: 1-5 requests of 0-6000 tokens, the GQA shape (Hq/Hkv 32/8, 16/8, 8/8,
16/4), 1-80 queries per request (so both matrix-core kernels: one 32-row tile or several),
bf16 or fp16, block 16/32/64, causal limits or none, a partial query count per request or
none, and a block table as wide as the longest request or twice that.  Tolerances as in
test_attention_gpu.py: lse atol 1e-4; out atol 2e-4 (the probabilities enter the P.V
product as a hi and a lo term in the cache dtype, about 16 significant bits).
"""
import math
import random

import pytest
import torch

from actkv.kernels.lse_attn import paged_decode_attention
from actkv.paged import PagedKVCache
from oracle import reference as ref

pytestmark = pytest.mark.gpu

GQA = [(32, 8), (16, 8), (8, 8), (16, 4)]


def _case(seed):
    rnd = random.Random(seed)
    n_req = rnd.randint(1, 5)
    lens = [rnd.choice([0, rnd.randint(1, 200), rnd.randint(200, 6000)]) for _ in range(n_req)]
    if max(lens) == 0:
        lens[0] = rnd.randint(1, 3000)
    hq, hkv = rnd.choice(GQA)
    return dict(lens=lens, hq=hq, hkv=hkv, n_q=rnd.choice([1, rnd.randint(2, 8), rnd.randint(9, 80)]),
                dtype=rnd.choice([torch.bfloat16, torch.float16]), bs=rnd.choice([16, 32, 64]),
                causal=rnd.random() < 0.5, partial=rnd.random() < 0.3, widen=rnd.choice([1, 2]))


@pytest.mark.parametrize("seed", range(64))
def test_random_shapes_match_the_oracle(seed):
    c = _case(seed)
    lens, hq, hkv, n_q, dtype, bs = c["lens"], c["hq"], c["hkv"], c["n_q"], c["dtype"], c["bs"]
    print(f"case {seed}: {c}", flush=True)
    g = torch.Generator().manual_seed(seed)
    nb = sum(math.ceil(n / bs) for n in lens) + 3
    cache = PagedKVCache(nb, bs, hkv, 128, n_layers=1, dtype=dtype, device="cuda")
    cache.free = torch.randperm(nb, generator=g).tolist()
    for r, n in enumerate(lens):
        cache.append(r, torch.randn(1, n, hkv, 128, generator=g).to(dtype).cuda(),
                     torch.randn(1, n, hkv, 128, generator=g).to(dtype).cuda())
    reqs = list(range(len(lens)))
    seq, bt = cache._device_tables(reqs)
    table = torch.zeros(len(lens), bt.shape[1] * c["widen"], dtype=torch.int32, device="cuda")
    table[:, : bt.shape[1]] = bt
    q = torch.randn(len(lens), n_q, hq, 128, generator=g).to(dtype)
    kv_len = (torch.stack([torch.randint(0, S + 4, (n_q,), generator=g) for S in lens]).to(torch.int32)
              if c["causal"] else None)
    n_valid = (torch.tensor([random.Random(seed + r).randint(0, n_q) for r in reqs], dtype=torch.int32)
               if c["partial"] else None)
    out, lse = paged_decode_attention(q.cuda(), cache.kv[0], table, seq,
                                      kv_len=None if kv_len is None else kv_len.cuda(),
                                      n_valid=None if n_valid is None else n_valid.cuda())
    want_out, want_lse = ref.paged_attention(
        q.float(), cache.kv[0].cpu().float(), [cache.tables[r] for r in reqs], [cache.seq_used[r] for r in reqs],
        kv_len=None if kv_len is None else kv_len.tolist(), n_valid=None if n_valid is None else n_valid.tolist())
    torch.testing.assert_close(lse.cpu(), want_lse, rtol=0, atol=1e-4)
    torch.testing.assert_close(out.cpu(), want_out, rtol=0, atol=2e-4)   # P as hi + lo terms


@pytest.mark.parametrize("seed", range(24))
def test_random_shapes_with_other_groups_match_the_oracle(seed):
    """The same sweep for groups of 3 and 5 to 8 query heads per KV head (Hq/Hkv 64/8, 16/2,
    8/1, 24/8, 40/8, 48/8, 28/4): decode tiles and multi-tile row groups."""
    rnd = random.Random(9000 + seed)
    n_req = rnd.randint(1, 4)
    lens = [rnd.choice([0, rnd.randint(1, 200), rnd.randint(200, 5000)]) for _ in range(n_req)]
    if max(lens) == 0:
        lens[0] = rnd.randint(1, 3000)
    hq, hkv = rnd.choice([(64, 8), (16, 2), (8, 1), (24, 8), (40, 8), (48, 8), (28, 4)])
    n_q = rnd.choice([1, rnd.randint(2, 4), rnd.randint(5, 60)])
    dtype, bs = rnd.choice([torch.bfloat16, torch.float16]), rnd.choice([16, 32, 64])
    causal, partial = rnd.random() < 0.5, rnd.random() < 0.3
    print(f"case {seed}: lens {lens} hq {hq} hkv {hkv} n_q {n_q} {dtype} bs {bs} causal {causal} "
          f"partial {partial}", flush=True)
    g = torch.Generator().manual_seed(7000 + seed)
    nb = sum(math.ceil(n / bs) for n in lens) + 3
    cache = PagedKVCache(nb, bs, hkv, 128, n_layers=1, dtype=dtype, device="cuda")
    cache.free = torch.randperm(nb, generator=g).tolist()
    for r, n in enumerate(lens):
        cache.append(r, torch.randn(1, n, hkv, 128, generator=g).to(dtype).cuda(),
                     torch.randn(1, n, hkv, 128, generator=g).to(dtype).cuda())
    reqs = list(range(len(lens)))
    seq, bt = cache._device_tables(reqs)
    q = torch.randn(len(lens), n_q, hq, 128, generator=g).to(dtype)
    kv_len = (torch.stack([torch.randint(0, S + 4, (n_q,), generator=g) for S in lens]).to(torch.int32)
              if causal else None)
    n_valid = (torch.tensor([random.Random(seed + r).randint(0, n_q) for r in reqs], dtype=torch.int32)
               if partial else None)
    out, lse = paged_decode_attention(q.cuda(), cache.kv[0], bt, seq,
                                      kv_len=None if kv_len is None else kv_len.cuda(),
                                      n_valid=None if n_valid is None else n_valid.cuda())
    want_out, want_lse = ref.paged_attention(
        q.float(), cache.kv[0].cpu().float(), [cache.tables[r] for r in reqs], [cache.seq_used[r] for r in reqs],
        kv_len=None if kv_len is None else kv_len.tolist(), n_valid=None if n_valid is None else n_valid.tolist())
    torch.testing.assert_close(lse.cpu(), want_lse, rtol=0, atol=1e-4)
    torch.testing.assert_close(out.cpu(), want_out, rtol=0, atol=2e-4)


@pytest.mark.parametrize("seed", range(24))
def test_random_shapes_at_head_dim_64_match_the_oracle(seed):
    """The same sweep at head dim 64 (Hq/Hkv 32/8, 64/8, 16/2, 8/8, 56/8): decode tiles and
    multi-tile row groups, blocks 16-64, a table up to twice as wide as the longest request."""
    rnd = random.Random(11000 + seed)
    n_req = rnd.randint(1, 4)
    lens = [rnd.choice([0, rnd.randint(1, 200), rnd.randint(200, 5000)]) for _ in range(n_req)]
    if max(lens) == 0:
        lens[0] = rnd.randint(1, 3000)
    hq, hkv = rnd.choice([(32, 8), (64, 8), (16, 2), (8, 8), (56, 8)])
    n_q = rnd.choice([1, rnd.randint(2, 4), rnd.randint(5, 60)])
    dtype, bs = rnd.choice([torch.bfloat16, torch.float16]), rnd.choice([16, 32, 64])
    causal, partial, widen = rnd.random() < 0.5, rnd.random() < 0.3, rnd.choice([1, 2])
    print(f"case {seed}: lens {lens} hq {hq} hkv {hkv} n_q {n_q} {dtype} bs {bs} causal {causal} "
          f"partial {partial} widen {widen}", flush=True)
    g = torch.Generator().manual_seed(13000 + seed)
    nb = sum(math.ceil(n / bs) for n in lens) + 3
    cache = PagedKVCache(nb, bs, hkv, 64, n_layers=1, dtype=dtype, device="cuda")
    cache.free = torch.randperm(nb, generator=g).tolist()
    for r, n in enumerate(lens):
        cache.append(r, torch.randn(1, n, hkv, 64, generator=g).to(dtype).cuda(),
                     torch.randn(1, n, hkv, 64, generator=g).to(dtype).cuda())
    reqs = list(range(len(lens)))
    seq, bt = cache._device_tables(reqs)
    table = torch.zeros(len(lens), bt.shape[1] * widen, dtype=torch.int32, device="cuda")
    table[:, : bt.shape[1]] = bt
    q = torch.randn(len(lens), n_q, hq, 64, generator=g).to(dtype)
    kv_len = (torch.stack([torch.randint(0, S + 4, (n_q,), generator=g) for S in lens]).to(torch.int32)
              if causal else None)
    n_valid = (torch.tensor([random.Random(seed + r).randint(0, n_q) for r in reqs], dtype=torch.int32)
               if partial else None)
    out, lse = paged_decode_attention(q.cuda(), cache.kv[0], table, seq,
                                      kv_len=None if kv_len is None else kv_len.cuda(),
                                      n_valid=None if n_valid is None else n_valid.cuda())
    want_out, want_lse = ref.paged_attention(
        q.float(), cache.kv[0].cpu().float(), [cache.tables[r] for r in reqs], [cache.seq_used[r] for r in reqs],
        kv_len=None if kv_len is None else kv_len.tolist(), n_valid=None if n_valid is None else n_valid.tolist())
    torch.testing.assert_close(lse.cpu(), want_lse, rtol=0, atol=1e-4)
    torch.testing.assert_close(out.cpu(), want_out, rtol=0, atol=2e-4)   # P as hi + lo terms


@pytest.mark.parametrize("seed", range(24))
def test_random_shapes_on_the_float32_path_match_the_oracle(seed):
    """Shapes off the matrix cores (head dims other than 64 and 128, float32 caches, blocks
    that are not a power of two from 16 up, groups up to 40): the float32 kernel's row groups
    and token split, against the oracle; out and lse within 1e-4."""
    rnd = random.Random(15000 + seed)
    n_req = rnd.randint(1, 4)
    lens = [rnd.choice([0, rnd.randint(1, 200), rnd.randint(200, 4000)]) for _ in range(n_req)]
    if max(lens) == 0:
        lens[0] = rnd.randint(1, 3000)
    d = rnd.choice([8, 30, 36, 80, 96, 256, 512])
    hkv = rnd.choice([1, 2, 4])
    hq = hkv * rnd.choice([1, 2, 3, 4, 8, rnd.randint(9, 40)])
    n_q = rnd.choice([1, rnd.randint(2, 4), rnd.randint(5, 24)])
    dtype, bs = rnd.choice([torch.bfloat16, torch.float16, torch.float32]), rnd.choice([8, 12, 16, 32])
    causal, partial = rnd.random() < 0.5, rnd.random() < 0.3
    print(f"case {seed}: lens {lens} d {d} hq {hq} hkv {hkv} n_q {n_q} {dtype} bs {bs} causal {causal} "
          f"partial {partial}", flush=True)
    g = torch.Generator().manual_seed(17000 + seed)
    nb = sum(math.ceil(n / bs) for n in lens) + 3
    cache = PagedKVCache(nb, bs, hkv, d, n_layers=1, dtype=dtype, device="cuda")
    cache.free = torch.randperm(nb, generator=g).tolist()
    for r, n in enumerate(lens):
        cache.append(r, torch.randn(1, n, hkv, d, generator=g).to(dtype).cuda(),
                     torch.randn(1, n, hkv, d, generator=g).to(dtype).cuda())
    reqs = list(range(len(lens)))
    seq, bt = cache._device_tables(reqs)
    q = torch.randn(len(lens), n_q, hq, d, generator=g).to(dtype)
    kv_len = (torch.stack([torch.randint(0, S + 4, (n_q,), generator=g) for S in lens]).to(torch.int32)
              if causal else None)
    n_valid = (torch.tensor([random.Random(seed + r).randint(0, n_q) for r in reqs], dtype=torch.int32)
               if partial else None)
    out, lse = paged_decode_attention(q.cuda(), cache.kv[0], bt, seq,
                                      kv_len=None if kv_len is None else kv_len.cuda(),
                                      n_valid=None if n_valid is None else n_valid.cuda())
    want_out, want_lse = ref.paged_attention(
        q.float(), cache.kv[0].cpu().float(), [cache.tables[r] for r in reqs], [cache.seq_used[r] for r in reqs],
        kv_len=None if kv_len is None else kv_len.tolist(), n_valid=None if n_valid is None else n_valid.tolist())
    torch.testing.assert_close(lse.cpu(), want_lse, rtol=0, atol=1e-4)
    torch.testing.assert_close(out.cpu(), want_out, rtol=0, atol=1e-4)
