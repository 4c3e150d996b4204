"""Parity at the workload sizes the eviction path is quoted on.

The one-layer 2k fp16 and 32k bf16 workloads fit the CPU oracle: scores are compared with the oracle's N reference folds
(rtol 1e-3, the float tolerance of the eviction path), the keep mask / perm / allocator lists /
every K-V byte bit-exactly with the oracle's evict on the GPU's own scores.
The 36-layer ragged batch and the 36-layer 131k sequence (tens of GB of K/V) are checked at full size through size-independent
properties -- the oracle's keep mask and plan on the GPU's scores, sequential allocator
semantics, survivors == pre-compaction rows at perm on every layer, untouched rows unchanged --
with every layer's and request's scores against a float32 torch reference on the GPU and
oracle spot checks of the scores on the smallest request."""
import math

import numpy as np
import pytest
import torch

from actkv.paged import PagedKVCache
from oracle import reference as ref

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.contiguous().view(torch.int16 if t.element_size() == 2 else torch.int32)


def _exact_lse_gpu(kv_layer, table, seq_used, q):
    """lse[n, h] = logsumexp_t scale q[n,h].k_t over the whole prefix, float32 on the GPU.
    kv_layer [2, NB, BS, Hkv, D] (device), q [N, Hq, D] (device)."""
    bs, hkv, d = kv_layer.shape[2], kv_layer.shape[3], kv_layer.shape[4]
    n_q, hq, _ = q.shape
    g = hq // hkv
    nblk = math.ceil(seq_used / bs)
    blocks = torch.tensor(table[:nblk], device=q.device, dtype=torch.long)
    k = kv_layer[0].index_select(0, blocks).reshape(-1, hkv, d)[:seq_used].float()
    lse = torch.empty(n_q, hq, device=q.device)
    for h in range(hkv):
        kt = k[:, h].t().contiguous()
        qh = q[:, h * g:(h + 1) * g].float().reshape(-1, d)
        lse[:, h * g:(h + 1) * g] = torch.logsumexp((qh @ kt) * d ** -0.5, -1).view(n_q, g)
    return lse


def _scores_fp32_gpu(kv_layer, table, seq_used, q, lse):
    """Float32 torch reference of one request's scores on the GPU (every layer and request of
    a large case, where the CPU oracle covers a sample): mean over the N action queries of
    max over the GQA group of exp(scale q.k - lse).  q [N, Hq, D], lse [N, Hq] (device);
    returns [Hkv, seq_used]."""
    bs, hkv, d = kv_layer.shape[2], kv_layer.shape[3], kv_layer.shape[4]
    n_q, hq, _ = q.shape
    g = hq // hkv
    nblk = math.ceil(seq_used / bs)
    blocks = torch.tensor(table[:nblk], device=q.device, dtype=torch.long)
    k = kv_layer[0].index_select(0, blocks).reshape(-1, hkv, d)[:seq_used].float()
    out = torch.empty(hkv, seq_used, device=q.device)
    for h in range(hkv):
        kt = k[:, h].t().contiguous()
        qh = q[:, h * g:(h + 1) * g].float().reshape(-1, d)
        p = torch.exp((qh @ kt) * d ** -0.5 - lse[:, h * g:(h + 1) * g].reshape(-1, 1))
        out[h] = p.view(n_q, g, seq_used).amax(1).mean(0)
    return out


def _single_layer_case(S, n_q, dtype, budget, sinks, seed):
    bs, hkv, hq, d = 16, 8, 32, 128
    g = torch.Generator().manual_seed(seed)
    nb = math.ceil(S / bs) + 16
    cache = PagedKVCache(nb, bs, hkv, d, n_layers=1, dtype=dtype, device="cuda")
    cache.free = torch.randperm(nb, generator=g).tolist()
    k = torch.randn(1, S, hkv, d, generator=g).to(dtype)
    v = torch.randn(1, S, hkv, d, generator=g).to(dtype)
    cache.append(0, k.cuda(), v.cuda())
    q = torch.randn(1, n_q, hq, d, generator=g).to(dtype)
    lse = _exact_lse_gpu(cache.kv[0], cache.tables[0], S, q[0].cuda()).unsqueeze(0)
    return cache, q, lse


@pytest.mark.parametrize("name,S,n_q,dtype,keep_frac", [
    ("1layer_2k_fp16", 2048, 64, torch.float16, 0.25),
    ("1layer_32k_bf16", 32768, 128, torch.bfloat16, 0.10),
])
def test_single_layer_configs_match_the_oracle(name, S, n_q, dtype, keep_frac):
    budget, sinks = int(keep_frac * S), 4
    cache, q, lse = _single_layer_case(S, n_q, dtype, budget, sinks, seed=S)
    width = math.ceil(S / 16) * 16
    out = torch.zeros(1, 8, width, device="cuda")
    n_seen = torch.zeros(1, dtype=torch.int32, device="cuda")
    cache.cal_attn([0], q.cuda(), lse, out, n_seen)
    # scores: N reference folds on the CPU
    want = torch.zeros(1, 8, width)
    ref.action_scores_nfold(q, cache.kv[0].cpu(), [cache.tables[0]], [S], lse.cpu(), want,
                            torch.zeros(1, dtype=torch.int32))
    torch.testing.assert_close(out.cpu(), want, rtol=1e-3, atol=1e-9)
    assert int(n_seen) == n_q
    # evict: keep mask, perm, K/V bytes, allocator lists, pins bit-exact with the oracle's
    # evict on the GPU's own scores
    model = ref.PagedCacheModel(cache.num_blocks, 16, 8, 128, 1)
    model.kv = _bits(cache.kv).cpu().numpy().copy()
    model.free, model.tables, model.seq_used = list(cache.free), {0: list(cache.tables[0])}, dict(cache.seq_used)
    scores = out[0]
    perm = cache.evict(0, scores, budget, protected=sinks)
    perm_o = model.evict(0, scores.cpu(), budget, protected=sinks, tie_rule="lowest")
    assert np.array_equal(perm.cpu().numpy(), perm_o)
    assert np.array_equal(_bits(cache.kv).cpu().numpy(), model.kv), "K/V bytes differ"
    assert cache.free == model.free and cache.tables == model.tables and cache.seq_used == model.seq_used
    assert np.array_equal(cache.pinned[0].cpu().numpy(), model.pinned[0])
    assert cache.seq_used[0] == budget + sinks


def _ragged_stack(seed, layers, lens, n_qs, dtype=torch.bfloat16, with_queries=True):
    bs, hkv, hq, d = 16, 8, 32, 128
    g = torch.Generator().manual_seed(seed)
    nb = sum(math.ceil(s / bs) for s in lens) + 64
    cache = PagedKVCache(nb, bs, hkv, d, n_layers=layers, dtype=dtype, device="cuda")
    cache.free = torch.randperm(nb, generator=g).tolist()      # one shuffled shared pool
    gd = torch.Generator(device="cuda").manual_seed(seed)
    for r, s in enumerate(lens):
        k = torch.randn(layers, s, hkv, d, generator=gd, device="cuda", dtype=dtype)
        v = torch.randn(layers, s, hkv, d, generator=gd, device="cuda", dtype=dtype)
        cache.append(r, k, v)
        del k, v
    if not with_queries:
        return cache, None, None
    n_max = max(n_qs)
    q = torch.randn(layers, len(lens), n_max, hq, d, generator=gd, device="cuda", dtype=dtype)
    lse = torch.zeros(layers, len(lens), n_max, hq, device="cuda")
    for l in range(layers):
        for r, s in enumerate(lens):
            lse[l, r, :n_qs[r]] = _exact_lse_gpu(cache.kv[l], cache.tables[r], s, q[l, r, :n_qs[r]])
    return cache, q, lse


def _allocator_after(free, tables, seq_used, reqs, keeps, bs):
    """Sequential evict semantics on the allocator lists (paged.py:135-138), in request order."""
    free, tables, seq_used = list(free), {r: list(t) for r, t in tables.items()}, dict(seq_used)
    for r, keep in zip(reqs, keeps):
        _, _, perm, drop = ref.plan_compaction(keep, seq_used[r], tables[r], bs)
        freed = tables[r][:drop]
        tables[r] = tables[r][drop:]
        free.extend(reversed(freed))
        seq_used[r] = int(perm.size)
    return free, tables, seq_used


def _check_moves(cache, before, slots_before, perms, plans, layers_to_check):
    """Survivors of every request == the pre-compaction rows at perm (per checked layer), and
    every row that is not a compaction destination is unchanged (all layers, K and V)."""
    bs, hkv, d = cache.block_size, cache.n_kv_heads, cache.head_dim
    for r, perm in perms.items():
        slots_after = cache.slot_map(r)
        for l in layers_to_check:
            fb = before[l].view(2, -1, hkv, d)
            fa = cache.kv[l].view(2, -1, hkv, d)
            assert torch.equal(_bits(fa[:, slots_after]), _bits(fb[:, slots_before[r][perm]])), (r, l)
    n_slots = cache.num_blocks * bs
    written = torch.zeros(n_slots, dtype=torch.bool, device="cuda")
    for src, dst in plans.values():
        written[torch.as_tensor(dst, device="cuda")] = True
    flat_a = cache.kv.view(cache.n_layers * 2, n_slots, hkv * d)
    flat_b = before.view(cache.n_layers * 2, n_slots, hkv * d)
    keep_idx = torch.nonzero(~written).flatten()
    for p in range(0, cache.n_layers * 2, 8):
        assert torch.equal(_bits(flat_a[p:p + 8].index_select(1, keep_idx)),
                           _bits(flat_b[p:p + 8].index_select(1, keep_idx))), "a non-destination row changed"


def test_36_layers_8_ragged_sequences_one_evict_call():
    """36 layers, 8 ragged sequences (8192..65536 tokens) in one shuffled pool, 64..256 action
    queries each, per-sequence keep ratio 0.05..0.30: score + keep + compact + reclaim of every
    request in one evict call (evict_batch == sequential evicts in request order)."""
    rng = np.random.default_rng(3)
    layers, R = 36, 8
    lens = [int(x) for x in rng.integers(8192, 65537, R)]
    n_qs = [int(x) for x in rng.integers(64, 257, R)]
    ratios = rng.uniform(0.05, 0.30, R)
    budgets = [int(ratios[r] * lens[r]) for r in range(R)]
    cache, q, lse = _ragged_stack(3, layers, lens, n_qs)
    reqs = list(range(R))
    width = max(len(cache.tables[r]) for r in reqs) * 16
    out = torch.zeros(layers, R, 8, width, device="cuda")
    n_seen = torch.zeros(R, dtype=torch.int32, device="cuda")
    n_valid = torch.tensor(n_qs, dtype=torch.int32, device="cuda")
    cache.cal_attn(reqs, q, lse, out, n_seen, layer=None, n_valid=n_valid)
    assert n_seen.tolist() == n_qs
    # every layer and request against the float32 torch reference on the GPU ...
    for l in range(layers):
        for r in reqs:
            want = _scores_fp32_gpu(cache.kv[l], cache.tables[r], lens[r], q[l, r, :n_qs[r]], lse[l, r, :n_qs[r]])
            torch.testing.assert_close(out[l, r, :, :lens[r]], want, rtol=1e-3, atol=1e-9, msg=f"layer {l} request {r}")
    # ... and the oracle's reference folds on the smallest request, two layers
    r0 = int(np.argmin(lens))
    for l in (0, layers - 1):
        want = torch.zeros(1, 8, width)
        ref.action_scores_nfold(q[l, r0:r0 + 1, :n_qs[r0]].cpu(), cache.kv[l].cpu(), [cache.tables[r0]], [lens[r0]],
                                lse[l, r0:r0 + 1, :n_qs[r0]].cpu(), want, torch.zeros(1, dtype=torch.int32))
        torch.testing.assert_close(out[l, r0].cpu(), want[0], rtol=1e-3, atol=1e-9)
    # evict every request in one call
    before = cache.kv.clone()
    slots_before = {r: cache.slot_map(r) for r in reqs}
    free0, tables0, seq0 = list(cache.free), {r: list(t) for r, t in cache.tables.items()}, dict(cache.seq_used)
    scores_cpu = out.cpu()
    keeps = [ref.keep_mask_lowest_index_ties(scores_cpu[:, r], lens[r], budgets[r], protected=4).numpy()
             for r in reqs]
    perms = cache.evict_batch(reqs, out, budgets, protected=4)
    torch.cuda.synchronize()
    plans = {}
    for r in reqs:
        src, dst, perm_o, _ = ref.plan_compaction(keeps[r], lens[r], tables0[r], 16)
        assert np.array_equal(perms[r].cpu().numpy(), perm_o), f"request {r}: perm differs"
        plans[r] = (src, dst)
    free_o, tables_o, seq_o = _allocator_after(free0, tables0, seq0, reqs, keeps, 16)
    assert cache.free == free_o and cache.tables == tables_o and cache.seq_used == seq_o
    _check_moves(cache, before, slots_before, {r: perms[r] for r in reqs}, plans, layers_to_check=range(layers))


def test_36_layers_131k_tokens_clustered_runs_compaction():
    """One 131072-token sequence, 36 layers; keep mask drawn as clustered runs (geometric run
    lengths, mean 32 kept / 128 dropped, overall keep ~0.2): plan, moves of all 72 planes and
    whole-block reclaim, against the oracle plan and the size-independent properties."""
    layers, S = 36, 131072
    cache, _, _ = _ragged_stack(4, layers, [S], [1], with_queries=False)
    rng = np.random.default_rng(4)
    keep = np.zeros(S, dtype=bool)
    t, on = 0, bool(rng.integers(0, 2))
    while t < S:
        run = int(rng.geometric(1 / 32 if on else 1 / 128))
        keep[t:t + run] = on
        t += run
        on = not on
    assert 0.1 < keep.mean() < 0.3
    before = cache.kv.clone()
    slots_before = {0: cache.slot_map(0)}
    free0, tables0, seq0 = list(cache.free), {0: list(cache.tables[0])}, dict(cache.seq_used)
    perm = cache.compact(0, torch.from_numpy(keep).cuda())
    torch.cuda.synchronize()
    src, dst, perm_o, drop = ref.plan_compaction(keep, S, tables0[0], 16)
    assert np.array_equal(perm.cpu().numpy(), perm_o)
    free_o, tables_o, seq_o = _allocator_after(free0, tables0, seq0, [0], [keep], 16)
    assert cache.free == free_o and cache.tables == tables_o and cache.seq_used == seq_o
    assert drop == math.ceil(S / 16) - math.ceil(int(keep.sum()) / 16)
    _check_moves(cache, before, slots_before, {0: perm}, {0: (src, dst)}, layers_to_check=range(layers))
