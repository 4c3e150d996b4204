"""Pin the CPU oracle (oracle/reference.py) independently of its own formulas: known answers of
the reference's tests, brute force from the definitions with plain Python loops, closed forms,
and torch's own CPU reductions.  Mutants of the oracle (a plausible mistake planted on the CPU)
must fail these checks, which shows the checks can see such mistakes."""
import math
import random

import numpy as np
import pytest
import torch

from oracle import reference as ref


# ----------------------------------------------------------------------------- helpers

def _cache(lens, bs=4, hkv=2, d=8, seed=0, dtype=torch.float32):
    """A paged K/V layer [2, NB, bs, hkv, d] with shuffled physical blocks, + tables."""
    g = torch.Generator().manual_seed(seed)
    nb = sum(math.ceil(n / bs) for n in lens) + 3
    kv = torch.randn(2, nb, bs, hkv, d, generator=g).to(dtype)
    order = torch.randperm(nb, generator=g).tolist()
    tables, i = [], 0
    for n in lens:
        k = math.ceil(n / bs)
        tables.append(order[i:i + k])
        i += k
    return kv, tables


def _k_row(kv, table, bs, t, h):
    return kv[0, table[t // bs], t % bs, h].double().tolist()


def _brute_scores(q_list, kv, table, seq_used, bs, scale, n_seen0=0, out0=None):
    """Running mean of max_g exp(scale q.k - lse) from the definition, float64 loops.
    q_list: list of [Hq][D] python lists (one per action query)."""
    hkv = kv.shape[3]
    hq = len(q_list[0])
    g = hq // hkv
    out = [[0.0] * seq_used for _ in range(hkv)] if out0 is None else [list(r) for r in out0]
    for n, q in enumerate(q_list):
        logits = [[scale * sum(a * b for a, b in zip(q[hh], _k_row(kv, table, bs, t, hh // g)))
                   for t in range(seq_used)] for hh in range(hq)]
        lse = [math.log(sum(math.exp(x) for x in row)) for row in logits]
        for h in range(hkv):
            for t in range(seq_used):
                p = max(math.exp(logits[h * g + j][t] - lse[h * g + j]) for j in range(g))
                out[h][t] += (p - out[h][t]) / (n_seen0 + n + 1)
    return out


# ----------------------------------------------------------------------------- scoring

def test_one_query_probabilities_sum_to_one():
    """Reference known answer (tests/test_kernels.py:58-66): Hq == Hkv, one query -> a softmax."""
    kv, tables = _cache([50], bs=16, hkv=1, d=16)
    q = torch.randn(1, 1, 16, generator=torch.Generator().manual_seed(1))
    lse = ref.decode_lse(q, kv, tables, [50])
    out = torch.zeros(1, 1, 64)
    ref.action_scores_fold(q, kv, tables, [50], lse, out, torch.zeros(1, dtype=torch.int32))
    assert abs(float(out[0, 0, :50].sum()) - 1.0) < 1e-5
    assert float(out[0, 0, 50:].abs().sum()) == 0.0


@pytest.mark.parametrize("hq,hkv,bs,S,n_q", [(4, 2, 4, 13, 3), (6, 3, 4, 9, 2), (2, 2, 8, 17, 4), (8, 2, 4, 7, 1)])
def test_folds_match_brute_force(hq, hkv, bs, S, n_q):
    d = 8
    kv, tables = _cache([S], bs=bs, hkv=hkv, d=d, seed=S)
    g = torch.Generator().manual_seed(hq)
    qs = [torch.randn(1, hq, d, generator=g) for _ in range(n_q)]
    out = torch.zeros(1, hkv, math.ceil(S / bs) * bs)
    n_seen = torch.zeros(1, dtype=torch.int32)
    for q in qs:
        lse = ref.decode_lse(q, kv, tables, [S])
        ref.action_scores_fold(q, kv, tables, [S], lse, out, n_seen)
    want = _brute_scores([q[0].tolist() for q in qs], kv, tables[0], S, bs, d ** -0.5)
    np.testing.assert_allclose(out[0, :, :S].numpy(), np.array(want), rtol=2e-5, atol=1e-9)
    assert int(n_seen) == n_q


def test_decode_lse_is_logsumexp():
    kv, tables = _cache([11], bs=4, hkv=2, d=8, seed=3)
    q = torch.randn(1, 4, 8, generator=torch.Generator().manual_seed(3))
    lse = ref.decode_lse(q, kv, tables, [11])
    for hh in range(4):
        logits = [8 ** -0.5 * sum(a * b for a, b in zip(q[0, hh].tolist(), _k_row(kv, tables[0], 4, t, hh // 2)))
                  for t in range(11)]
        assert abs(float(lse[0, hh]) - math.log(sum(math.exp(x) for x in logits))) < 1e-5


def test_running_mean_is_the_arithmetic_mean():
    kv, tables = _cache([40], bs=8, hkv=2, d=16, seed=4)
    g = torch.Generator().manual_seed(4)
    q = torch.randn(1, 7, 8, 16, generator=g)
    lse = torch.stack([ref.decode_lse(q[:, n], kv, tables, [40]) for n in range(7)], 1)
    out = torch.zeros(1, 2, 40)
    ref.action_scores_nfold(q, kv, tables, [40], lse, out, torch.zeros(1, dtype=torch.int32))
    singles = []
    for n in range(7):
        o = torch.zeros(1, 2, 40)
        ref.action_scores_fold(q[:, n], kv, tables, [40], lse[:, n], o, torch.zeros(1, dtype=torch.int32))
        singles.append(o)
    torch.testing.assert_close(out, torch.stack(singles).mean(0), rtol=1e-5, atol=1e-9)


def test_group_heads_sharing_q_and_lse_reduce_to_one_head():
    """G = 4 query heads holding the same q (hence the same lse): the group max is that head."""
    kv, tables = _cache([30], bs=4, hkv=2, d=8, seed=5)
    q1 = torch.randn(1, 2, 8, generator=torch.Generator().manual_seed(5))
    q4 = q1.repeat_interleave(4, dim=1)
    lse1, lse4 = ref.decode_lse(q1, kv, tables, [30]), ref.decode_lse(q4, kv, tables, [30])
    o1, o4 = torch.zeros(1, 2, 32), torch.zeros(1, 2, 32)
    ref.action_scores_fold(q1, kv, tables, [30], lse1, o1, torch.zeros(1, dtype=torch.int32))
    ref.action_scores_fold(q4, kv, tables, [30], lse4, o4, torch.zeros(1, dtype=torch.int32))
    torch.testing.assert_close(o1, o4, rtol=1e-6, atol=0)


def test_scores_do_not_depend_on_the_physical_block_order():
    kv, tables = _cache([37], bs=4, hkv=2, d=8, seed=6)
    perm = torch.randperm(kv.shape[1], generator=torch.Generator().manual_seed(6))
    kv2 = torch.empty_like(kv)
    kv2[:, perm] = kv
    tables2 = [[int(perm[b]) for b in tables[0]]]
    q = torch.randn(1, 4, 8, generator=torch.Generator().manual_seed(7))
    lse = ref.decode_lse(q, kv, tables, [37])
    o1, o2 = torch.zeros(1, 2, 40), torch.zeros(1, 2, 40)
    ref.action_scores_fold(q, kv, tables, [37], lse, o1, torch.zeros(1, dtype=torch.int32))
    ref.action_scores_fold(q, kv2, tables2, [37], lse, o2, torch.zeros(1, dtype=torch.int32))
    assert torch.equal(o1, o2)


def test_nfold_with_ragged_counts_and_causal_limits_matches_brute_force():
    bs, S, hq, hkv, d = 4, 14, 4, 2, 8
    kv, tables = _cache([S, S], bs=bs, hkv=hkv, d=d, seed=8)
    g = torch.Generator().manual_seed(8)
    n_q = 3
    q = torch.randn(2, n_q, hq, d, generator=g)
    lse = torch.stack([ref.decode_lse(q[:, n], kv, tables, [S, S]) for n in range(n_q)], 1)
    n_valid = torch.tensor([3, 2], dtype=torch.int32)
    kv_len = torch.tensor([[5, 14, 9], [1, 7, 14]], dtype=torch.int32)
    out = torch.zeros(2, hkv, 16)
    n_seen = torch.tensor([1, 0], dtype=torch.int32)
    out[0, :, :S] = 0.25
    ref.action_scores_nfold(q, kv, tables, [S, S], lse, out, n_seen, n_valid=n_valid, kv_len=kv_len)
    for r in range(2):
        o = [[0.25 if r == 0 else 0.0] * S for _ in range(hkv)]
        n0 = 1 if r == 0 else 0
        for n in range(int(n_valid[r])):
            qq = q[r, n].tolist()
            logits = [[d ** -0.5 * sum(a * b for a, b in zip(qq[hh], _k_row(kv, tables[r], bs, t, hh // 2)))
                       for t in range(S)] for hh in range(hq)]
            for h in range(hkv):
                for t in range(S):
                    p = 0.0
                    if t < int(kv_len[r, n]):
                        p = max(math.exp(logits[h * 2 + j][t] - float(lse[r, n, h * 2 + j])) for j in range(2))
                    o[h][t] += (p - o[h][t]) / (n0 + n + 1)
        np.testing.assert_allclose(out[r, :, :S].numpy(), np.array(o), rtol=2e-5, atol=1e-9)
    assert n_seen.tolist() == [4, 2]


@pytest.mark.parametrize("mutant", ["mean_over_group", "sum_over_group", "no_lse", "no_scale",
                                    "fold_denominator"])
def test_a_planted_scoring_mistake_is_caught(monkeypatch, mutant):
    """Each mutant restates one plausible mistake; the brute-force check must reject it."""
    orig = ref._group_probs

    def group_probs(q_r, k, lse_r, scale, reduce="amax", use_lse=True):
        hkv = k.shape[1]
        g = q_r.shape[0] // hkv
        kk = k.float().repeat_interleave(g, dim=1)
        logits = torch.einsum("hd,shd->hs", q_r.float(), kk) * scale
        p = torch.exp(logits - lse_r.unsqueeze(-1) if use_lse else logits)
        return getattr(p.view(hkv, g, -1), reduce)(1)

    if mutant == "mean_over_group":
        monkeypatch.setattr(ref, "_group_probs", lambda q, k, l, s: group_probs(q, k, l, s, "mean"))
    elif mutant == "sum_over_group":
        monkeypatch.setattr(ref, "_group_probs", lambda q, k, l, s: group_probs(q, k, l, s, "sum"))
    elif mutant == "no_lse":
        monkeypatch.setattr(ref, "_group_probs", lambda q, k, l, s: group_probs(q, k, l, s, use_lse=False))
    elif mutant == "no_scale":
        monkeypatch.setattr(ref, "_group_probs", lambda q, k, l, s: orig(q, k, l, 1.0))
    else:
        def bad_fold(q, kv_layer, table, seq_used, lse, out, n_seen, scale=None):
            scale = q.shape[-1] ** -0.5 if scale is None else scale
            p = ref._group_probs(q[0], ref.gather_k(kv_layer, table[0], int(seq_used[0])), lse[0], scale)
            cur = out[0, :, :int(seq_used[0])]
            out[0, :, :int(seq_used[0])] = cur + (p - cur) / (float(n_seen[0]) + 2.0)
            n_seen += 1
        monkeypatch.setattr(ref, "action_scores_fold", bad_fold)
    with pytest.raises(AssertionError):
        test_folds_match_brute_force(4, 2, 4, 13, 3)


# ----------------------------------------------------------------------------- keep mask

def test_keep_mask_known_answer_head_reduce():
    """Reference known answer (tests/test_kernels.py:178-183)."""
    scores = torch.zeros(2, 2, 4)
    scores[0, 0, 1] = 1.0
    scores[:, :, 2] = 0.3
    assert ref.keep_mask_from_scores(scores, 4, budget=1).tolist() == [False, False, True, False]
    assert ref.keep_mask_from_scores(scores, 4, budget=1, head_reduce="max").tolist() == [False, True, False, False]
    with pytest.raises(ValueError):
        ref.keep_mask_from_scores(scores, 4, budget=1, head_reduce="sum")


@pytest.mark.parametrize("seed", range(6))
def test_keep_mask_matches_a_sort_of_float64_means(seed):
    """Protected prefix + the top-budget others by (mean over layers of mean/max over heads)."""
    rng = random.Random(seed)
    L, H, S = rng.randint(1, 5), rng.randint(1, 4), rng.randint(5, 60)
    budget, prot = rng.randint(0, S), rng.randint(0, 5)
    g = torch.Generator().manual_seed(seed)
    scores = torch.randperm(L * H * S, generator=g).float().view(L, H, S) / (L * H * S)
    for reduce in ("mean", "max"):
        per = [[(max if reduce == "max" else (lambda v: sum(v) / len(v)))([float(scores[l, h, t]) for h in range(H)])
                for t in range(S)] for l in range(L)]
        s = [sum(per[l][t] for l in range(L)) / L for t in range(S)]
        cand = [t for t in range(S) if t >= prot]
        top = sorted(cand, key=lambda t: (-s[t], t))[:max(0, min(budget, len(cand)))]
        want = [t < prot or t in top for t in range(S)]
        got = ref.keep_mask_from_scores(scores, S, budget, protected=prot, head_reduce=reduce)
        assert got.tolist() == want


@pytest.mark.parametrize("L,H,S,W", [(36, 8, 4096, 4096), (36, 8, 1000, 1024), (1, 8, 333, 333), (20, 8, 640, 700),
                                     (40, 16, 97, 128), (3, 3, 65, 65), (300, 8, 256, 256), (36, 32, 70, 96)])
def test_torch_cpu_mean_order_is_the_documented_one(L, H, S, W):
    """torch's CPU float32 mean == the cascade / row_sum order the device reduction follows
    (bit for bit), for the head mean and the layer mean, at every column."""
    g = torch.Generator().manual_seed(L + S)
    x = (torch.rand(L, H, W, generator=g) * torch.exp(torch.randn(L, H, W, generator=g) * 3)).float()[..., :S]
    m1 = x.mean(-2)
    want1 = np.stack([ref.torch_mean_emulation(x[l].numpy(), S) for l in range(L)])
    assert np.array_equal(m1.numpy().view(np.uint32), want1.view(np.uint32))
    m2 = m1.reshape(-1, S).mean(0)
    want2 = ref.torch_mean_emulation(m1.numpy(), S)
    assert np.array_equal(m2.numpy().view(np.uint32), want2.view(np.uint32))


def test_lowest_index_tie_rule():
    scores = torch.zeros(1, 1, 20)
    scores[0, 0, [3, 9, 15]] = 2.0
    scores[0, 0, [1, 4, 8, 12, 19]] = 1.0
    keep = ref.keep_mask_lowest_index_ties(scores, 20, 5, protected=2)
    assert torch.nonzero(keep).flatten().tolist() == [0, 1, 3, 4, 8, 9, 15]


# ----------------------------------------------------------------------------- compaction plan

@pytest.mark.parametrize("seed", range(40))
def test_plan_matches_brute_force(seed):
    rng = random.Random(seed)
    bs = rng.choice([1, 2, 4, 8, 16])
    S = rng.randint(0, 70)
    keep = [rng.random() < rng.choice([0.05, 0.3, 0.7, 1.0]) for _ in range(S)]
    table = list(range(math.ceil(S / bs) + 3))
    rng.shuffle(table)
    src, dst, perm, drop = ref.plan_compaction(np.array(keep, dtype=bool), S, table, bs)
    bsrc, bdst, bperm, bdrop = ref.plan_compaction_bruteforce(keep, S, table, bs)
    assert src.tolist() == bsrc and dst.tolist() == bdst and perm.tolist() == bperm and drop == bdrop


@pytest.mark.parametrize("seq_used,budget,bs", [(100, 40, 16), (17, 10, 16), (64, 64, 16), (200, 3, 8), (33, 0, 16)])
def test_plan_invariants(seq_used, budget, bs):
    """Reference invariants (tests/test_kernels.py:80-91)."""
    g = torch.Generator().manual_seed(seq_used)
    keep = torch.zeros(seq_used, dtype=torch.bool)
    keep[torch.randperm(seq_used, generator=g)[:budget]] = True
    table = torch.randperm(math.ceil(seq_used / bs) + 4, generator=g)
    src, dst, perm, drop = ref.plan_compaction(keep.numpy(), seq_used, table.numpy(), bs)
    assert not (set(src.tolist()) & set(dst.tolist()))
    assert len(set(src.tolist())) == len(src) and len(set(dst.tolist())) == len(dst)
    assert sorted(perm.tolist()) == torch.nonzero(keep).flatten().tolist()
    assert drop == math.ceil(seq_used / bs) - math.ceil(budget / bs)


def test_apply_copies_is_a_row_memcpy():
    flat = np.arange(4 * 300 * 6, dtype=np.uint16).reshape(4, 300, 6)
    before = flat.copy()
    src, dst = [3, 50, 77, 299], [10, 11, 200, 0]
    ref.apply_copies(flat, src, dst)
    for p in range(4):
        for s, d in zip(src, dst):
            assert np.array_equal(flat[p, d], before[p, s])
    untouched = [i for i in range(300) if i not in dst]
    assert np.array_equal(flat[:, untouched], before[:, untouched])


# ----------------------------------------------------------------------------- paged cache model

def _model(lens, bs=16, hkv=2, d=16, layers=1, seed=0):
    g = torch.Generator().manual_seed(seed)
    nb = sum(math.ceil(n / bs) for n in lens) + 8
    m = ref.PagedCacheModel(nb, bs, hkv, d, layers, np_dtype=np.float32)
    m.free = torch.randperm(nb, generator=g).tolist()
    for r, n in enumerate(lens):
        k = torch.randn(layers, n, hkv, d, generator=g).numpy()
        v = torch.randn(layers, n, hkv, d, generator=g).numpy()
        m.append(r, k, v)
    return m


@pytest.mark.parametrize("n,budget", [(150, 60), (40, 39), (33, 16)])
def test_model_compaction_preserves_kept_entries_and_frees_blocks(n, budget):
    """Reference known answer (tests/test_kernels.py:122-135)."""
    m = _model([n], layers=2)
    before = [m.gather(0, layer)[0].copy() for layer in range(2)]
    used = m.used_blocks
    keep = np.zeros(n, dtype=bool)
    keep[torch.randperm(n, generator=torch.Generator().manual_seed(n))[:budget].numpy()] = True
    perm = m.compact(0, keep)
    assert m.seq_used[0] == budget
    for layer in range(2):
        assert np.array_equal(m.gather(0, layer)[0], before[layer][perm])
    assert used - m.used_blocks == math.ceil(n / 16) - math.ceil(budget / 16)


def test_model_evict_known_answer():
    """Reference known answer (tests/test_kernels.py:157-168)."""
    m = _model([70], hkv=2, d=16, layers=2)
    scores = 0.1 * torch.rand(2, 2, 70, generator=torch.Generator().manual_seed(3))
    hot = [5, 17, 40, 69]
    scores[..., hot] += 1.0
    perm = m.evict(0, scores, budget=4, protected=3)
    assert sorted(perm.tolist()) == [0, 1, 2, *hot]
    assert m.seq_used[0] == 7 and len(m.tables[0]) == 1


def test_model_evict_within_budget_and_repeated_evictions():
    """Reference known answers (tests/test_kernels.py:171-175 and :186-200)."""
    m = _model([20])
    table = list(m.tables[0])
    assert m.evict(0, torch.rand(2, 20), budget=20).tolist() == list(range(20))
    assert m.tables[0] == table and m.seq_used[0] == 20
    m = _model([64])
    prompt = m.gather(0)[0][:8].copy()
    scores = torch.zeros(2, 64)
    scores[:, 8:56] = torch.rand(2, 48, generator=torch.Generator().manual_seed(4)) + 1
    m.evict(0, scores, budget=24, protected=8)
    new = torch.randn(1, 16, 2, 16, generator=torch.Generator().manual_seed(5)).numpy()
    m.append(0, new, new)
    scores = torch.zeros(2, m.seq_used[0])
    scores[:, -16:] = 1.0
    m.evict(0, scores, budget=16, protected=8)
    k = m.gather(0)[0]
    assert m.seq_used[0] == 24
    assert all(any(np.array_equal(p, row) for row in k) for p in prompt)


def test_model_free_list_is_a_stack():
    m = ref.PagedCacheModel(6, 2, 1, 1, 1, np_dtype=np.float32)
    m.append(0, np.zeros((1, 5, 1, 1), np.float32), np.zeros((1, 5, 1, 1), np.float32))
    assert m.tables[0] == [0, 1, 2] and m.free == [5, 4, 3]
    # B = 2, Y = 3, X = 1: window [4, 6); slot 4 stays, 5 (past S) is the hole that
    # receives the kept token 2; logical blocks 0 and 1 are dropped
    keep = np.array([False, False, True, False, True])
    perm = m.compact(0, keep)
    assert perm.tolist() == [4, 2]
    assert m.tables[0] == [2] and m.seq_used[0] == 2
    # dropped blocks go back reversed: the first freed block is popped next
    assert m.free == [5, 4, 3, 1, 0]


def test_model_append_and_slot_map_known_answer():
    """Blocks are popped from the end of the free stack as each append needs them and token
    t lives at table[t // bs] * bs + t % bs (paged.py:67-84, :93-97)."""
    m = ref.PagedCacheModel(6, 2, 1, 1, 2, np_dtype=np.float32)
    m.free = [3, 0, 5, 1, 4, 2]
    tok = np.arange(1, 8, dtype=np.float32).reshape(1, 7, 1, 1)
    m.append(7, np.concatenate([tok[:, :3]] * 2), -np.concatenate([tok[:, :3]] * 2))
    assert m.tables[7] == [2, 4] and m.free == [3, 0, 5, 1]
    m.append(7, np.concatenate([tok[:, 3:]] * 2), -np.concatenate([tok[:, 3:]] * 2))
    assert m.tables[7] == [2, 4, 1, 5] and m.free == [3, 0] and m.seq_used[7] == 7
    assert m.slot_map(7).tolist() == [4, 5, 8, 9, 2, 3, 10]
    flat = m.kv.reshape(2, 2, 12)
    for layer in range(2):
        assert flat[layer, 0, [4, 5, 8, 9, 2, 3, 10]].tolist() == list(range(1, 8))
        assert flat[layer, 1, [4, 5, 8, 9, 2, 3, 10]].tolist() == [-t for t in range(1, 8)]
    assert flat[:, :, [0, 1, 6, 7, 11]].sum() == 0
    k, v = m.gather(7, layer=1)
    assert k.ravel().tolist() == list(range(1, 8)) and v.ravel().tolist() == [-t for t in range(1, 8)]


# ---------------------------------------------------------------- LRFU keep score

def test_top_p_mask_known_answer():
    """tests/test_algorithms.py:16-19 of the reference."""
    s = torch.tensor([0.5, 0.05, 0.3, 0.15, 0.0])
    assert ref.top_p_mask(s, 0.9).tolist() == [True, False, True, True, False]
    assert ref.top_p_mask(s, 0.9, stable=True).tolist() == [True, False, True, True, False]


@pytest.mark.parametrize("seed", range(20))
def test_top_p_mask_matches_brute_force(seed):
    g = torch.Generator().manual_seed(seed)
    n = int(torch.randint(1, 60, (1,), generator=g))
    x = torch.rand(n, generator=g) ** 3
    x[torch.rand(n, generator=g) < 0.2] = 0.0
    if seed % 4 == 0:                                  # ties
        x = torch.round(x * 8) / 8
    p = float(torch.rand(1, generator=g)) * 0.98 + 0.01
    assert ref.top_p_mask(x, p, stable=True).tolist() == ref.top_p_mask_bruteforce(x, p)


def test_top_p_mask_edge_cases():
    assert ref.top_p_mask(torch.zeros(0), 0.9).tolist() == []
    assert ref.top_p_mask(torch.zeros(4), 0.9).tolist() == [False] * 4
    assert ref.top_p_mask(torch.tensor([0.0, 2.0, 0.0]), 0.5).tolist() == [False, True, False]
    assert ref.top_p_mask(torch.tensor([1.0, 1.0, 1.0]), 1.0, stable=True).tolist() == [True] * 3


def test_lrfu_update_known_answers():
    """tests/test_algorithms.py:22-48 of the reference (Algorithm 1 update, and a round without
    an action region only decays)."""
    ks = torch.zeros(4)
    ref.lrfu_update(ks, torch.tensor([0.05, 0.05, 0.8, 0.1]), 4, 0, 0.5, 0.9)
    torch.testing.assert_close(ks, torch.tensor([0.0, 0.0, 0.8, 0.1]))
    ks2 = torch.cat([ks, torch.zeros(2)])
    ref.lrfu_update(ks2, torch.tensor([0.0, 0.0, 0.0, 0.05, 0.95, 0.0]), 6, 0, 0.5, 0.9)
    torch.testing.assert_close(ks2, torch.tensor([0.0, 0.0, 0.4, 0.05, 0.95, 0.0]))
    ks3 = torch.cat([ks, torch.zeros(2)])
    ref.lrfu_update(ks3, torch.zeros(6), 6, 0, 0.5, 0.9, active=False)
    torch.testing.assert_close(ks3, torch.tensor([0.0, 0.0, 0.4, 0.05, 0.0, 0.0]))


def test_paged_lrfu_update_with_a_prefix_equals_the_reference_form():
    g = torch.Generator().manual_seed(3)
    act = torch.rand(3, 50, generator=g)
    ks_a = torch.rand(3, 50, generator=g)
    ks_b = ks_a.clone()
    ref.paged_lrfu_update(ks_a, act, 50, 6, 0.5, 0.9, stable=False)
    for l in range(3):
        ref.lrfu_update(ks_b[l], act[l], 50, 6, 0.5, 0.9)
    assert torch.equal(ks_a, ks_b)
    # a pinned mask equal to the prefix gives the same result
    ks_c = ks_b.clone()
    ks_d = ks_b.clone()
    pin = torch.arange(50) < 6
    ref.paged_lrfu_update(ks_c, act, 50, pin, 0.5, 0.9)
    ref.paged_lrfu_update(ks_d, act, 50, 6, 0.5, 0.9)
    assert torch.equal(ks_c, ks_d)


def test_top_p_mask_total_orders_agree_away_from_the_boundary():
    """The float64-rounded total (the device's) and torch's float32 total give the same nucleus
    unless a running sum lies within a few ulps of p * total: on random heavy-tailed inputs the
    masks agree almost always, and where they differ the boundary is that close."""
    g = torch.Generator().manual_seed(9)
    differ = 0
    for _ in range(300):
        x = (torch.rand(2000, generator=g) ** 8) * 1e-2
        a = ref.top_p_mask(x, 0.9, stable=True)
        b = ref.top_p_mask(x, 0.9, stable=True, total64=True)
        if not torch.equal(a, b):
            differ += 1
            vals = torch.sort(x, descending=True, stable=True).values
            csum = torch.cumsum(vals, 0)
            thr_a, thr_b = 0.9 * x.sum(), 0.9 * x.double().sum().float()
            lo, hi = min(float(thr_a), float(thr_b)), max(float(thr_a), float(thr_b))
            assert bool(((csum >= lo) & (csum <= hi)).any())
    assert differ <= 30


# ---------------------------------------------------------------- paged attention (lse producer)

def _v_row(kv, table, bs, t, h):
    return kv[1, table[t // bs], t % bs, h].double().tolist()


def test_paged_attention_matches_the_definition():
    """out and lse from float64 loops over the definition (lse_attn.py:42-60): GQA 2, two
    queries per request, causal limits, ragged requests."""
    bs, hkv, d = 4, 2, 8
    kv, tables = _cache([11, 6], bs=bs, hkv=hkv, d=d, seed=21)
    g = torch.Generator().manual_seed(22)
    q = torch.randn(2, 2, 4, d, generator=g)
    kv_len = [[5, 11], [6, 3]]
    out, lse = ref.paged_attention(q, kv, tables, [11, 6], kv_len=kv_len)
    scale = d ** -0.5
    for r, S in enumerate([11, 6]):
        for n in range(2):
            lim = min(kv_len[r][n], S)
            for hh in range(4):
                logits = [scale * sum(a * b for a, b in zip(q[r, n, hh].tolist(), _k_row(kv, tables[r], bs, t, hh // 2)))
                          for t in range(lim)]
                m = max(logits)
                w = [math.exp(x - m) for x in logits]
                z = sum(w)
                assert abs(float(lse[r, n, hh]) - (m + math.log(z))) < 1e-5
                want = [sum(w[t] * _v_row(kv, tables[r], bs, t, hh // 2)[j] for t in range(lim)) / z for j in range(d)]
                assert max(abs(a - b) for a, b in zip(out[r, n, hh].tolist(), want)) < 1e-5


def test_paged_attention_known_answers():
    """Equal keys give a uniform softmax: out = mean of the V rows, lse = logit + log S; one
    token gives out = v_0; no token gives lse = -inf, out = 0; rows past n_valid stay 0."""
    bs, hkv, d = 4, 1, 8
    kv, tables = _cache([7], bs=bs, hkv=hkv, d=d, seed=23)
    kv[0] = 0.5                                                    # every key equal
    q = torch.ones(1, 3, 1, d)
    out, lse = ref.paged_attention(q, kv, tables, [7], kv_len=[[7, 1, 0]])
    logit = d ** -0.5 * 0.5 * d
    vs = torch.stack([torch.tensor(_v_row(kv, tables[0], bs, t, 0), dtype=torch.float64) for t in range(7)])
    assert abs(float(lse[0, 0, 0]) - (logit + math.log(7))) < 1e-5
    torch.testing.assert_close(out[0, 0, 0].double(), vs.mean(0), rtol=1e-6, atol=1e-6)
    assert abs(float(lse[0, 1, 0]) - logit) < 1e-6
    torch.testing.assert_close(out[0, 1, 0].double(), vs[0], rtol=1e-6, atol=1e-6)
    assert float(lse[0, 2, 0]) == -math.inf and torch.equal(out[0, 2, 0], torch.zeros(d))
    out2, lse2 = ref.paged_attention(q, kv, tables, [7], n_valid=[2])
    assert torch.equal(out2[0, 2], torch.zeros(1, d)) and float(lse2[0, 2, 0]) == 0.0


def test_paged_attention_lse_is_decode_lse_and_normalises():
    """One query per request without limits: lse equals decode_lse (pinned above), and the
    recovered probabilities exp(s - lse) sum to 1 over the tokens."""
    kv, tables = _cache([13, 30], bs=4, hkv=2, d=16, seed=24)
    q = torch.randn(2, 1, 8, 16, generator=torch.Generator().manual_seed(25))
    out, lse = ref.paged_attention(q, kv, tables, [13, 30])
    torch.testing.assert_close(lse[:, 0], ref.decode_lse(q[:, 0], kv, tables, [13, 30]), rtol=0, atol=1e-6)
    for r, S in enumerate([13, 30]):
        k = ref.gather_k(kv, tables[r], S).double().repeat_interleave(4, dim=1)
        s = torch.einsum("hd,shd->hs", q[r, 0].double(), k) * 16 ** -0.5
        tot = torch.exp(s - lse[r, 0].double().unsqueeze(-1)).sum(-1)
        torch.testing.assert_close(tot, torch.ones(8, dtype=torch.float64), rtol=0, atol=1e-6)
