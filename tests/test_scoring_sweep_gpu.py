"""Action-query scoring (actkv_action_scores through action_scores) over a seeded random sweep
of shapes, against the oracle's fold of lse_attn.py:63-78 (action_scores_nfold).

Each case draws: 1-5 requests of 1-6000 tokens, the GQA shape (Hq/Hkv 32/8, 16/8, 8/8: groups
4, 2, 1 on the matrix cores), 1-150 action queries (more than 512/G rows run as several
launches), bf16 or fp16, block 16/32/64, causal limits or none, a partial query count per
request or none, and running means with earlier counts n_seen.  Bar: scores rtol 1e-3, the
scoring bar; n_seen exact.
"""
import math
import random

import pytest
import torch

from actkv.kernels.lse_attn import action_scores
from actkv.paged import PagedKVCache
from oracle import reference as ref

pytestmark = pytest.mark.gpu

GQA = [(32, 8), (16, 8), (8, 8)]


def _case(seed):
    rnd = random.Random(1000 + seed)
    n_req = rnd.randint(1, 5)
    return dict(lens=[rnd.choice([rnd.randint(1, 300), rnd.randint(300, 6000)]) for _ in range(n_req)],
                gqa=rnd.choice(GQA), n_q=rnd.choice([1, rnd.randint(2, 40), rnd.randint(41, 150)]),
                dtype=rnd.choice([torch.bfloat16, torch.float16]), bs=rnd.choice([16, 32, 64]),
                causal=rnd.random() < 0.5, partial=rnd.random() < 0.3)


@pytest.mark.parametrize("seed", range(32))
def test_random_shapes_match_the_oracle(seed):
    c = _case(seed)
    lens, (hq, hkv), n_q, dtype, bs = c["lens"], c["gqa"], c["n_q"], c["dtype"], c["bs"]
    print(f"case {seed}: {c}", flush=True)
    g = torch.Generator().manual_seed(seed)
    nb = sum(math.ceil(n / bs) for n in lens) + 3
    cache = PagedKVCache(nb, bs, hkv, 128, n_layers=1, dtype=dtype, device="cuda")
    cache.free = torch.randperm(nb, generator=g).tolist()
    for r, n in enumerate(lens):
        cache.append(r, torch.randn(1, n, hkv, 128, generator=g).to(dtype).cuda(),
                     torch.randn(1, n, hkv, 128, generator=g).to(dtype).cuda())
    reqs = list(range(len(lens)))
    bt, seq = cache.block_table(reqs), cache.seq_tensor(reqs)
    width = bt.shape[1] * bs
    q = torch.randn(len(reqs), n_q, hq, 128, generator=g).to(dtype)
    kv0 = cache.kv[0].cpu()
    tables = [cache.tables[r] for r in reqs]
    lse = torch.stack([ref.decode_lse(q[:, n], kv0, tables, lens) for n in range(n_q)], 1)
    kv_len = (torch.stack([torch.randint(1, s + 1, (n_q,), generator=g) for s in lens]).to(torch.int32)
              if c["causal"] else None)
    n_valid = (torch.tensor([random.Random(seed + r).randint(0, n_q) for r in reqs], dtype=torch.int32)
               if c["partial"] else None)
    out0 = torch.rand(len(reqs), hkv, width, generator=g)
    n0 = torch.randint(0, 9, (len(reqs),), generator=g).to(torch.int32)
    out_k, n_k = out0.cuda(), n0.cuda()
    action_scores(q.cuda(), cache.kv[0], bt, seq, lse.cuda(), out_k, n_k,
                  n_valid=None if n_valid is None else n_valid.cuda(),
                  kv_len=None if kv_len is None else kv_len.cuda())
    out_o, n_o = out0.clone(), n0.clone()
    ref.action_scores_nfold(q, kv0, tables, lens, lse, out_o, n_o, n_valid=n_valid, kv_len=kv_len)
    torch.testing.assert_close(out_k.cpu(), out_o, rtol=1e-3, atol=1e-6)
    assert torch.equal(n_k.cpu(), n_o)


def _case8(seed):
    rnd = random.Random(5000 + seed)
    n_req = rnd.randint(1, 4)
    return dict(lens=[rnd.choice([rnd.randint(1, 300), rnd.randint(300, 4000)]) for _ in range(n_req)],
                gqa=rnd.choice([(64, 8), (16, 2), (8, 1), (24, 8), (40, 8), (48, 8), (28, 4)]),
                n_q=rnd.choice([1, rnd.randint(2, 16), rnd.randint(17, 90)]),
                dtype=rnd.choice([torch.bfloat16, torch.float16]), bs=rnd.choice([16, 32, 64]),
                causal=rnd.random() < 0.5, partial=rnd.random() < 0.3)


@pytest.mark.parametrize("seed", range(24))
def test_random_shapes_with_other_groups_match_the_oracle(seed):
    """The same sweep for groups of 3 and 5 to 8 query heads per KV head (64/8, 16/2, 8/1, 24/8,
    40/8, 48/8, 28/4): more than 512/G' queries (G' the group padded to 4 or 8) run as several
    launches."""
    c = _case8(seed)
    lens, (hq, hkv), n_q, dtype, bs = c["lens"], c["gqa"], c["n_q"], c["dtype"], c["bs"]
    print(f"case {seed}: {c}", flush=True)
    g = torch.Generator().manual_seed(100 + seed)
    nb = sum(math.ceil(n / bs) for n in lens) + 3
    cache = PagedKVCache(nb, bs, hkv, 128, n_layers=1, dtype=dtype, device="cuda")
    cache.free = torch.randperm(nb, generator=g).tolist()
    for r, n in enumerate(lens):
        cache.append(r, torch.randn(1, n, hkv, 128, generator=g).to(dtype).cuda(),
                     torch.randn(1, n, hkv, 128, generator=g).to(dtype).cuda())
    reqs = list(range(len(lens)))
    bt, seq = cache.block_table(reqs), cache.seq_tensor(reqs)
    width = bt.shape[1] * bs
    q = torch.randn(len(reqs), n_q, hq, 128, generator=g).to(dtype)
    kv0 = cache.kv[0].cpu()
    tables = [cache.tables[r] for r in reqs]
    lse = torch.stack([ref.decode_lse(q[:, n], kv0, tables, lens) for n in range(n_q)], 1)
    kv_len = (torch.stack([torch.randint(1, s + 1, (n_q,), generator=g) for s in lens]).to(torch.int32)
              if c["causal"] else None)
    n_valid = (torch.tensor([random.Random(seed + r).randint(0, n_q) for r in reqs], dtype=torch.int32)
               if c["partial"] else None)
    out0 = torch.rand(len(reqs), hkv, width, generator=g)
    n0 = torch.randint(0, 9, (len(reqs),), generator=g).to(torch.int32)
    out_k, n_k = out0.cuda(), n0.cuda()
    action_scores(q.cuda(), cache.kv[0], bt, seq, lse.cuda(), out_k, n_k,
                  n_valid=None if n_valid is None else n_valid.cuda(),
                  kv_len=None if kv_len is None else kv_len.cuda())
    out_o, n_o = out0.clone(), n0.clone()
    ref.action_scores_nfold(q, kv0, tables, lens, lse, out_o, n_o, n_valid=n_valid, kv_len=kv_len)
    torch.testing.assert_close(out_k.cpu(), out_o, rtol=1e-3, atol=1e-6)
    assert torch.equal(n_k.cpu(), n_o)


@pytest.mark.parametrize("seed", range(12))
def test_random_shapes_with_groups_above_eight_match_the_oracle(seed):
    """Groups of 9 to 16 query heads per KV head (laid out as 16 rows per query): 128/8, 96/8,
    72/8, 32/2; more than 32 queries run as several launches."""
    rnd = random.Random(8000 + seed)
    n_req = rnd.randint(1, 3)
    lens = [rnd.choice([rnd.randint(1, 300), rnd.randint(300, 3000)]) for _ in range(n_req)]
    hq, hkv = rnd.choice([(128, 8), (96, 8), (72, 8), (32, 2)])
    n_q = rnd.choice([1, rnd.randint(2, 16), rnd.randint(17, 70)])
    dtype, bs = rnd.choice([torch.bfloat16, torch.float16]), rnd.choice([16, 32])
    causal, partial = rnd.random() < 0.5, rnd.random() < 0.3
    print(f"case {seed}: lens {lens} hq {hq} hkv {hkv} n_q {n_q} {dtype} bs {bs} causal {causal} "
          f"partial {partial}", flush=True)
    g = torch.Generator().manual_seed(300 + seed)
    nb = sum(math.ceil(n / bs) for n in lens) + 3
    cache = PagedKVCache(nb, bs, hkv, 128, n_layers=1, dtype=dtype, device="cuda")
    cache.free = torch.randperm(nb, generator=g).tolist()
    for r, n in enumerate(lens):
        cache.append(r, torch.randn(1, n, hkv, 128, generator=g).to(dtype).cuda(),
                     torch.randn(1, n, hkv, 128, generator=g).to(dtype).cuda())
    reqs = list(range(len(lens)))
    bt, seq = cache.block_table(reqs), cache.seq_tensor(reqs)
    width = bt.shape[1] * bs
    q = torch.randn(len(reqs), n_q, hq, 128, generator=g).to(dtype)
    kv0 = cache.kv[0].cpu()
    tables = [cache.tables[r] for r in reqs]
    lse = torch.stack([ref.decode_lse(q[:, n], kv0, tables, lens) for n in range(n_q)], 1)
    kv_len = (torch.stack([torch.randint(1, s + 1, (n_q,), generator=g) for s in lens]).to(torch.int32)
              if causal else None)
    n_valid = (torch.tensor([random.Random(seed + r).randint(0, n_q) for r in reqs], dtype=torch.int32)
               if partial else None)
    out0 = torch.rand(len(reqs), hkv, width, generator=g)
    n0 = torch.randint(0, 9, (len(reqs),), generator=g).to(torch.int32)
    out_k, n_k = out0.cuda(), n0.cuda()
    action_scores(q.cuda(), cache.kv[0], bt, seq, lse.cuda(), out_k, n_k,
                  n_valid=None if n_valid is None else n_valid.cuda(),
                  kv_len=None if kv_len is None else kv_len.cuda())
    out_o, n_o = out0.clone(), n0.clone()
    ref.action_scores_nfold(q, kv0, tables, lens, lse, out_o, n_o, n_valid=n_valid, kv_len=kv_len)
    torch.testing.assert_close(out_k.cpu(), out_o, rtol=1e-3, atol=1e-6)
    assert torch.equal(n_k.cpu(), n_o)


def _generic_case(seed):
    """Shapes off the matrix cores: head dims other than 64 and 128 (30 and 90 not multiples of 4:
    the row-at-a-time kernel), float32 caches or queries, groups up to 96, any block size."""
    rnd = random.Random(5000 + seed)
    d = rnd.choice([8, 24, 30, 36, 80, 90, 96, 160, 256, 512])
    hkv = rnd.choice([1, 2])
    g_max = 96 if d <= 96 else 16
    g = rnd.choice([1, 3, 4, 5, rnd.randint(6, g_max)])
    qdt, kdt = rnd.choice([(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                           (torch.float16, torch.float16), (torch.float32, torch.bfloat16)])
    return dict(lens=[rnd.randint(1, 1500) for _ in range(rnd.randint(1, 3))], d=d, hq=g * hkv, hkv=hkv,
                n_q=rnd.choice([1, rnd.randint(2, 12), rnd.randint(13, 30)]), qdt=qdt, kdt=kdt,
                bs=rnd.choice([8, 12, 16, 32]), causal=rnd.random() < 0.5, partial=rnd.random() < 0.3)


@pytest.mark.parametrize("seed", range(24))
def test_random_shapes_on_the_float32_path_match_the_oracle(seed):
    c = _generic_case(seed)
    lens, d, hq, hkv, n_q, bs = c["lens"], c["d"], c["hq"], c["hkv"], c["n_q"], c["bs"]
    print(f"case {seed}: {c}", flush=True)
    g = torch.Generator().manual_seed(6000 + seed)
    nb = sum(math.ceil(n / bs) for n in lens) + 3
    cache = PagedKVCache(nb, bs, hkv, d, n_layers=1, dtype=c["kdt"], device="cuda")
    cache.free = torch.randperm(nb, generator=g).tolist()
    for r, n in enumerate(lens):
        cache.append(r, torch.randn(1, n, hkv, d, generator=g).to(c["kdt"]).cuda(),
                     torch.randn(1, n, hkv, d, generator=g).to(c["kdt"]).cuda())
    reqs = list(range(len(lens)))
    bt, seq = cache.block_table(reqs), cache.seq_tensor(reqs)
    width = bt.shape[1] * bs
    q = (torch.randn(len(reqs), n_q, hq, d, generator=g) * 0.5).to(c["qdt"])
    kv0 = cache.kv[0].cpu()
    tables = [cache.tables[r] for r in reqs]
    lse = torch.stack([ref.decode_lse(q[:, n].float(), kv0, tables, lens) for n in range(n_q)], 1)
    kv_len = (torch.stack([torch.randint(1, s + 1, (n_q,), generator=g) for s in lens]).to(torch.int32)
              if c["causal"] else None)
    n_valid = (torch.tensor([random.Random(seed + r).randint(0, n_q) for r in reqs], dtype=torch.int32)
               if c["partial"] else None)
    out0 = torch.rand(len(reqs), hkv, width, generator=g)
    n0 = torch.randint(0, 9, (len(reqs),), generator=g).to(torch.int32)
    out_k, n_k = out0.cuda(), n0.cuda()
    action_scores(q.cuda(), cache.kv[0], bt, seq, lse.cuda(), out_k, n_k,
                  n_valid=None if n_valid is None else n_valid.cuda(), kv_len=None if kv_len is None else kv_len.cuda())
    out_o, n_o = out0.clone(), n0.clone()
    ref.action_scores_nfold(q.float(), kv0, tables, lens, lse, out_o, n_o, n_valid=n_valid, kv_len=kv_len)
    rtol = 1e-4 if c["kdt"] == torch.float32 and c["qdt"] == torch.float32 else 1e-3
    torch.testing.assert_close(out_k.cpu(), out_o, rtol=rtol, atol=1e-6)
    assert torch.equal(n_k.cpu(), n_o)
