"""Device LRFU keep score (actkv_lrfu_update through actkv.kernels.lrfu) against the oracle's
restatement of eviction.py:36-50 / :209-218, and a small agent loop (append, causal action
scoring, LRFU keep + compaction) against the oracle paged-cache model."""
import math

import numpy as np
import pytest
import torch

from actkv.kernels.lrfu import LRFUConfig, PagedLRFU, lrfu_update
from actkv.paged import PagedKVCache
from oracle import reference as ref

pytestmark = pytest.mark.gpu


def test_known_answers_of_the_reference():
    """tests/test_algorithms.py:22-48 of the reference, through the device kernel."""
    ks = torch.zeros(1, 1, 8, device="cuda")
    sc = torch.zeros(1, 1, 1, 8, device="cuda")
    sc[0, 0, 0, :4] = torch.tensor([0.05, 0.05, 0.8, 0.1])
    lrfu_update(sc, ks, [4], 0, True, 0.5, 0.9)
    torch.testing.assert_close(ks[0, 0, :4].cpu(), torch.tensor([0.0, 0.0, 0.8, 0.1]))
    sc.zero_()
    sc[0, 0, 0, :6] = torch.tensor([0.0, 0.0, 0.0, 0.05, 0.95, 0.0])
    lrfu_update(sc, ks, [6], 0, True, 0.5, 0.9)
    torch.testing.assert_close(ks[0, 0, :6].cpu(), torch.tensor([0.0, 0.0, 0.4, 0.05, 0.95, 0.0]))
    lrfu_update(sc, ks, [6], 0, False, 0.5, 0.9)      # a round without an action region
    torch.testing.assert_close(ks[0, 0, :6].cpu(), torch.tensor([0.0, 0.0, 0.2, 0.025, 0.475, 0.0]))


@pytest.mark.parametrize("L,H,seqs,prots,W,reduce,p", [
    (3, 8, [1000, 1717], [4, 0], 1760, "mean", 0.9),
    (2, 4, [33, 300, 65], [5, 7, 0], 320, "max", 0.5),
    (36, 8, [4096], [4], 4096, "mean", 0.9),
    (1, 2, [50000], [4], 50016, "mean", 0.99),             # scores through the workspace
    (2, 8, [16384, 9000], [4, 0], 16384, "mean", 0.9),      # 16 tokens per thread in registers, full
    (3, 8, [4, 5, 6, 7, 3, 1, 9], [0, 1, 0, 2, 0, 0, 0], 40, "mean", 0.9),  # torch's 4-column body of 4-7 tokens
])
def test_lrfu_update_matches_the_oracle(L, H, seqs, prots, W, reduce, p):
    g = torch.Generator().manual_seed(sum(seqs))
    R = len(seqs)
    # action scores shaped like running means of probabilities (heavy-tailed, some zeros)
    scores = (torch.rand(L, R, H, W, generator=g) ** 8) * 1e-2
    scores[torch.rand(L, R, H, W, generator=g) < 0.05] = 0.0
    ks0 = torch.rand(L, R, W, generator=g) * 1e-3
    active = [True] * R
    if R > 1:
        active[1] = False
    ks = ks0.clone().cuda()
    hits = lrfu_update(scores.cuda(), ks, seqs, prots, active, 0.5, p, reduce, return_hits=True)
    ks_o = ks0.clone()
    for r in range(R):
        act = ref.paged_lrfu_act(scores[:, r], seqs[r], reduce)
        ks_row = ks_o[:, r]
        h_o = ref.paged_lrfu_update(ks_row, act, seqs[r], prots[r], 0.5, p, active[r], stable=True, total64=True)
        P = prots[r]
        assert torch.equal(hits[:, r, P:seqs[r]].cpu(), h_o[:, P:]), f"request {r}: hits differ"
    assert torch.equal(ks.cpu(), ks_o), "keep scores differ"


def test_lrfu_update_with_pinned_masks_and_ties():
    """Scattered pinned tokens are left out and keep their score; equal action scores at the
    crossing are taken lowest index first."""
    g = torch.Generator().manual_seed(5)
    L, R, H, W = 2, 2, 1, 200
    scores = torch.full((L, R, H, W), 0.01)
    scores[:, :, :, ::7] = 0.05
    scores[:, 1, :, 100:] = 0.0
    pinned = torch.rand(R, W, generator=g) < 0.1
    ks0 = torch.rand(L, R, W, generator=g)
    ks = ks0.clone().cuda()
    hits = lrfu_update(scores.cuda(), ks, [200, 150], pinned.cuda(), True, 0.5, 0.6, return_hits=True)
    ks_o = ks0.clone()
    for r, s in enumerate([200, 150]):
        act = ref.paged_lrfu_act(scores[:, r], s)
        h_o = ref.paged_lrfu_update(ks_o[:, r], act, s, pinned[r], 0.5, 0.6, True, stable=True, total64=True)
        assert torch.equal(hits[:, r, :s].cpu(), h_o)
    assert torch.equal(ks.cpu(), ks_o)
    assert torch.equal(ks.cpu()[:, pinned], ks0[:, pinned])


def _lse(cache, layer, req, q, kv_len):
    """lse[n, h] over tokens t < kv_len[n], float32 on the GPU (paged_decode_attention_ref
    semantics, causal per query)."""
    bs, hkv, d = cache.block_size, cache.n_kv_heads, cache.head_dim
    S = cache.seq_used[req]
    k = cache.gather(req, layer)[0].float()                  # [S, Hkv, D]
    n_q, hq, _ = q.shape
    g = hq // hkv
    logits = torch.einsum("nhgd,shd->nhgs", q.float().view(n_q, hkv, g, d), k) * d ** -0.5
    mask = torch.arange(S, device=q.device)[None, :] < kv_len[:, None]
    logits = logits.masked_fill(~mask[:, None, None, :], float("-inf"))
    return torch.logsumexp(logits, -1).reshape(n_q, hq)


def test_agent_loop_rounds_match_the_oracle():
    """A few rounds of the ORA loop on a small cache: each round appends observation,
    reasoning and action tokens to every request, scores the action tokens causally, then
    LRFU keep + compaction; KV bytes, tables, free list, pins and keep scores match the
    oracle run round by round."""
    torch.manual_seed(0)
    layers, hkv, hq, d, bs = 2, 2, 4, 128, 16
    reqs = [0, 1, 2]
    nb = 160
    cache = PagedKVCache(nb, bs, hkv, d, n_layers=layers, dtype=torch.bfloat16, device="cuda")
    g = torch.Generator().manual_seed(1)
    cache.free = torch.randperm(nb, generator=g).tolist()
    model = ref.PagedCacheModel(nb, bs, hkv, d, layers)
    model.free = list(cache.free)
    cap = 1200
    lr = PagedLRFU(cache, reqs, cap, LRFUConfig(decay=0.5, top_p=0.9))
    ks_o = torch.zeros(layers, len(reqs), cap)
    rng = np.random.default_rng(2)
    for rnd in range(4):
        n_act = []
        for r in reqs:
            n_new = int(rng.integers(60, 140))
            k = torch.randn(layers, n_new, hkv, d, generator=g).to(torch.bfloat16)
            v = torch.randn(layers, n_new, hkv, d, generator=g).to(torch.bfloat16)
            cache.append(r, k.cuda(), v.cuda())
            model.append(r, k.view(torch.int16).numpy().view(np.uint16), v.view(torch.int16).numpy().view(np.uint16))
            n_act.append(int(rng.integers(4, 12)) if not (rnd == 2 and r == 1) else 0)
        lr.begin_round()
        width = lr.scores.shape[-1]
        N = max(n_act)
        q = torch.randn(layers, len(reqs), N, hq, d, generator=g).to(torch.bfloat16).cuda()
        kv_len = torch.zeros(len(reqs), N, dtype=torch.int32)
        for j, r in enumerate(reqs):
            S = cache.seq_used[r]
            kv_len[j, :n_act[j]] = torch.arange(S - n_act[j] + 1, S + 1)   # action token j sees itself
        kv_len = kv_len.cuda()
        lse = torch.zeros(layers, len(reqs), N, hq, device="cuda")
        for l in range(layers):
            for j, r in enumerate(reqs):
                if n_act[j]:
                    lse[l, j, : n_act[j]] = _lse(cache, l, r, q[l, j, : n_act[j]], kv_len[j, : n_act[j]])
        cache.cal_attn(reqs, q, lse, lr.scores, lr.n_seen, layer=None,
                       n_valid=torch.tensor(n_act, dtype=torch.int32, device="cuda"), kv_len=kv_len)
        scores = lr.scores.cpu()
        budget = 150 + 40 * rnd
        perms = lr.evict(budget, protected=4, n_action=n_act)
        # oracle: same scores, LRFU update, keep = protected + top-budget of the layer mean
        for j, r in enumerate(reqs):
            S = model.seq_used[r]
            act = ref.paged_lrfu_act(scores[:, j], S)
            pin = model.pinned.get(r)
            pins = 4 if pin is None else torch.from_numpy(np.concatenate([pin, np.zeros(S - pin.size, bool)]))
            ref.paged_lrfu_update(ks_o[:, j], act, S, pins, 0.5, 0.9, n_act[j] > 0, stable=True, total64=True)
            perm_o = model.evict(r, ks_o[:, j, :S][:, None, :], budget, protected=4, tie_rule="lowest")
            assert np.array_equal(perms[j].cpu().numpy(), perm_o), (rnd, r)
            b = perm_o.size
            if b != S:
                ks_o[:, j, :b] = ks_o[:, j, torch.from_numpy(perm_o)]
                ks_o[:, j, b:] = 0.0
        assert torch.equal(lr.ks.cpu(), ks_o), f"round {rnd}: keep scores differ"
        kv = cache.kv.cpu().contiguous().view(torch.int16).numpy()
        assert np.array_equal(kv.view(np.uint16), model.kv), f"round {rnd}: KV bytes differ"
        assert cache.free == model.free and cache.tables == model.tables and cache.seq_used == model.seq_used
        for r in reqs:
            if r in model.pinned:
                assert np.array_equal(cache.pinned[r].cpu().numpy(), model.pinned[r])


@pytest.mark.parametrize("seed", range(24))
def test_lrfu_update_random_shapes_match_the_oracle(seed):
    """Seeded random shapes: 1-5 requests of 1-20000 tokens (some past the 16-per-thread
    register path), 1-4 layers, 1-8 heads, table width up to twice the longest request,
    mean or max head reduction, top_p 0.5-0.99, decay 0.3-0.9, protected prefixes, inactive
    requests, score vectors with zeros and exact ties; keep scores and hits bit-exact."""
    import random
    rnd = random.Random(3000 + seed)
    R = rnd.randint(1, 5)
    seqs = [rnd.choice([rnd.randint(1, 64), rnd.randint(64, 4096), rnd.randint(4096, 20000)]) for _ in range(R)]
    L, H = rnd.randint(1, 4), rnd.choice([1, 2, 4, 8])
    W = max(seqs) + rnd.choice([0, rnd.randint(1, max(seqs))])
    prots = [rnd.randint(0, min(s, 8)) for s in seqs]
    active = [rnd.random() < 0.8 for _ in seqs]
    reduce, p, decay = rnd.choice(["mean", "max"]), rnd.choice([0.5, 0.9, 0.99]), rnd.choice([0.3, 0.5, 0.9])
    g = torch.Generator().manual_seed(seed)
    scores = (torch.rand(L, R, H, W, generator=g) ** 8) * 1e-2
    scores[torch.rand(L, R, H, W, generator=g) < 0.05] = 0.0
    scores[torch.rand(L, R, H, W, generator=g) < 0.02] = 1e-3          # exact ties
    ks0 = torch.rand(L, R, W, generator=g) * 1e-3
    ks = ks0.clone().cuda()
    hits = lrfu_update(scores.cuda(), ks, seqs, prots, active, decay, p, reduce, return_hits=True)
    ks_o = ks0.clone()
    for r in range(R):
        act = ref.paged_lrfu_act(scores[:, r], seqs[r], reduce)
        h_o = ref.paged_lrfu_update(ks_o[:, r], act, seqs[r], prots[r], decay, p, active[r], stable=True,
                                    total64=True)
        assert torch.equal(hits[:, r, prots[r]:seqs[r]].cpu(), h_o[:, prots[r]:]), f"request {r}: hits differ"
    assert torch.equal(ks.cpu(), ks_o), "keep scores differ"
