"""The agent-loop (ORA) workload at its real shape, against the oracle, round by round.

Shape: a Qwen3-8B-shaped cache (36 layers, Hq 32 / Hkv 8, head_dim 128, block 16, bf16)
holding a batch of 4 sequences.  Each round appends, per sequence, U[512, 2048] observation
+ U[128, 512] reasoning + U[32, 64] action tokens (one batched append launch), scores the
action tokens causally (their lse from the paged attention kernel), updates the LRFU keep
score (decay 0.5, top-p 0.9; actkv/eviction.py:36-50, :198-224), keeps 4 sinks plus the top
`budget` tokens by the layer-average keep score with the budget on the 50-round schedule
4096 -> 16384, and compacts (actkv/paged.py:141-157).  Two stretches of that schedule are
run: its first 6 rounds (the sequences pass the budget from round 2 on, so blocks are
reclaimed), and its last 3 (budgets 15882-16384) on sequences pre-filled with 16000 tokens
each, the length the loop's sequences reach by then.

Checked after every round:
- scores of layers 0, 17 and 35 against the oracle's N reference folds (rtol 1e-3);
- keep scores of all 36 layers bit-exact against the oracle's LRFU update on the GPU's own
  scores (the device nucleus rule: equal scores lowest index first, float64 total);
- perm, block tables, free list, seq_used and pins bit-exact against the oracle paged cache;
- every K/V byte of layers 0, 17 and 35 bit-exact against the oracle cache (which holds
  those layers), so survivors sit where the plan puts them and no other row changed;
- layer 9 (not held by the oracle): each request's rows after the round equal its rows
  before the compaction at perm.
The compaction launches run with ACTKV_DEBUG=1, so the kernel's per-request report (kept,
moved, dropped, remaining blocks) and the plan's disjointness are checked as well.
"""

import numpy as np
import pytest
import torch

from actkv.kernels.lrfu import LRFUConfig, PagedLRFU
from actkv.paged import PagedKVCache
from oracle import reference as ref

pytestmark = pytest.mark.gpu

L, HKV, HQ, D, BS, R = 36, 8, 32, 128, 16, 4
HELD = (0, 17, 35)          # layers the oracle cache holds
PROBE = 9                   # a layer checked through the survivors-at-perm property
ROUNDS, SCHEDULE = 6, 50
B_LO, B_HI, SINKS = 4096, 16384, 4


def _u16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _budget(rnd):
    return int(round(B_LO + (B_HI - B_LO) * rnd / (SCHEDULE - 1)))


def _run_rounds(monkeypatch, rounds, prefill=0):
    """The agent loop over the schedule's `rounds` (indices into the 50-round schedule), each
    sequence first holding `prefill` tokens of history (appended, never scored)."""
    monkeypatch.setenv("ACTKV_DEBUG", "1")
    # a request holds at most its history or its last kept count (budget + sinks), plus one
    # round of appends
    cap = ((max(prefill, _budget(rounds[-1]) + SINKS) + 2624 + BS - 1) // BS) * BS
    nb = R * (cap // BS + 2) + 64
    gcpu = torch.Generator().manual_seed(5 + rounds[0])
    cache = PagedKVCache(nb, BS, HKV, D, n_layers=L, dtype=torch.bfloat16, device="cuda")
    cache.free = torch.randperm(nb, generator=gcpu).tolist()
    model = ref.PagedCacheModel(nb, BS, HKV, D, len(HELD))
    model.free = list(cache.free)
    gdev = torch.Generator(device="cuda").manual_seed(6 + rounds[0])
    rng = np.random.default_rng(7 + rounds[0])
    reqs = list(range(R))
    lr = PagedLRFU(cache, reqs, cap, LRFUConfig(decay=0.5, top_p=0.9))
    ks_o = torch.zeros(L, R, lr.width)
    held = torch.tensor(HELD, device="cuda")
    if prefill:
        k = torch.randn(L, R * prefill, HKV, D, generator=gdev, device="cuda", dtype=torch.bfloat16)
        v = torch.randn(L, R * prefill, HKV, D, generator=gdev, device="cuda", dtype=torch.bfloat16)
        cache.append_batch(reqs, k, v, [prefill] * R)
        kh, vh = _u16(k.index_select(0, held)), _u16(v.index_select(0, held))
        for j, r in enumerate(reqs):
            model.append(r, kh[:, j * prefill:(j + 1) * prefill], vh[:, j * prefill:(j + 1) * prefill])
        del k, v
        assert cache.tables == model.tables and cache.free == model.free, "prefill allocation"
    reclaimed = 0
    for rnd in rounds:
        budget = _budget(rnd)
        n_act, counts = [], []
        for _ in reqs:
            n_new = int(rng.integers(512, 2049)) + int(rng.integers(128, 513))
            a = int(rng.integers(32, 65))
            n_act.append(a)
            counts.append(n_new + a)
        k = torch.randn(L, sum(counts), HKV, D, generator=gdev, device="cuda", dtype=torch.bfloat16)
        v = torch.randn(L, sum(counts), HKV, D, generator=gdev, device="cuda", dtype=torch.bfloat16)
        cache.append_batch(reqs, k, v, counts)
        kh, vh = _u16(k.index_select(0, held)), _u16(v.index_select(0, held))
        off = 0
        for r, c in zip(reqs, counts):
            model.append(r, kh[:, off:off + c], vh[:, off:off + c])
            off += c
        del k, v
        assert cache.tables == model.tables and cache.free == model.free, f"round {rnd}: append allocation"
        seqs = [cache.seq_used[r] for r in reqs]
        nmax = max(n_act)
        q = torch.randn(L, R, nmax, HQ, D, generator=gdev, device="cuda", dtype=torch.bfloat16)
        kv_len = torch.zeros(R, nmax, dtype=torch.int32)
        for j, s in enumerate(seqs):
            kv_len[j, : n_act[j]] = torch.arange(s - n_act[j] + 1, s + 1)     # action token j sees itself
        kv_len_d = kv_len.cuda()
        n_valid = torch.tensor(n_act, dtype=torch.int32, device="cuda")
        _, lse = cache.decode_attention(reqs, q, layer=None, n_valid=n_valid, kv_len=kv_len_d)
        lr.begin_round()
        cache.cal_attn(reqs, q, lse, lr.scores, lr.n_seen, layer=None, n_valid=n_valid, kv_len=kv_len_d)
        scores = lr.scores.cpu()
        assert lr.n_seen.cpu().tolist() == n_act

        # scores of the held layers: the oracle's N reference folds on the oracle cache's K
        q_c, lse_c = q.cpu(), lse.cpu()
        tables = [model.tables[r] for r in reqs]
        for i, l in enumerate(HELD):
            kv_l = torch.from_numpy(model.kv[i].view(np.int16)).view(torch.bfloat16)
            want = torch.zeros(R, HKV, lr.width)
            ref.action_scores_nfold(q_c[l], kv_l, tables, seqs, lse_c[l], want, torch.zeros(R, dtype=torch.int32),
                                    n_valid=n_act, kv_len=kv_len)
            torch.testing.assert_close(scores[l], want, rtol=1e-3, atol=1e-9,
                                       msg=lambda m: f"round {rnd}, layer {l}: scores differ\n{m}")

        probe_before = [torch.cat(cache.gather(r, PROBE)).clone() for r in reqs]
        free_before = len(cache.free)
        perms = lr.evict(budget, protected=SINKS, n_action=n_act)
        reclaimed += len(cache.free) - free_before

        # oracle: LRFU update on the same scores, then keep + compaction of the oracle cache
        for j, r in enumerate(reqs):
            S = seqs[j]
            act = ref.paged_lrfu_act(scores[:, j], S)
            pin = model.pinned.get(r)
            pins = SINKS if pin is None else torch.from_numpy(np.concatenate([pin, np.zeros(S - pin.size, bool)]))
            ref.paged_lrfu_update(ks_o[:, j], act, S, pins, 0.5, 0.9, n_act[j] > 0, stable=True, total64=True)
            perm_o = model.evict(r, ks_o[:, j, :S][:, None, :], budget, protected=SINKS, tie_rule="lowest")
            assert np.array_equal(perms[j].cpu().numpy(), perm_o), f"round {rnd}, request {r}: perm differs"
            b = perm_o.size
            if b != S:
                ks_o[:, j, :b] = ks_o[:, j, torch.from_numpy(perm_o)]
                ks_o[:, j, b:] = 0.0
            after = torch.cat(cache.gather(r, PROBE))
            idx = perms[j]
            want_rows = torch.cat([probe_before[j][:S][idx], probe_before[j][S:][idx]])
            assert torch.equal(after.view(torch.int16), want_rows.view(torch.int16)), \
                f"round {rnd}, request {r}: layer {PROBE} survivors are not the rows at perm"
        assert torch.equal(lr.ks.cpu(), ks_o), f"round {rnd}: keep scores differ"
        kv_held = _u16(cache.kv.index_select(0, held))
        assert np.array_equal(kv_held, model.kv), f"round {rnd}: K/V bytes of layers {HELD} differ"
        assert cache.free == model.free and cache.tables == model.tables and cache.seq_used == model.seq_used, \
            f"round {rnd}: allocator state differs"
        for r in reqs:
            if r in model.pinned:
                assert np.array_equal(cache.pinned[r].cpu().numpy(), model.pinned[r]), f"round {rnd}: pins of {r}"
        print(f"round {rnd}: budget {budget}, {seqs} -> {[cache.seq_used[r] for r in reqs]} tokens, "
              f"{len(cache.free) - free_before} blocks reclaimed", flush=True)
    assert reclaimed > 0, "no round went over its budget"
    assert all(cache.seq_used[r] <= _budget(rounds[-1]) + SINKS for r in reqs)


def test_agent_loop_36_layers_batch_4_matches_the_oracle(monkeypatch):
    """The schedule's first 6 rounds on empty sequences."""
    _run_rounds(monkeypatch, list(range(ROUNDS)))


def test_agent_loop_late_schedule_matches_the_oracle(monkeypatch):
    """The schedule's last 3 rounds (budgets 15882, 16133, 16384) on sequences holding 16000
    tokens of history, as the loop's sequences do by round 47."""
    _run_rounds(monkeypatch, [SCHEDULE - 3, SCHEDULE - 2, SCHEDULE - 1], prefill=16000)
