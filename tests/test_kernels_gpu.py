"""HIP kernels vs the CPU oracle on the reference's kernel-test cases (tests/test_kernels.py of
the reference repository), plus the bf16/fp16 MFMA shapes.  Every call goes through the C ABI
(libactkv_hip.so) via the drop-in modules."""
import math

import numpy as np
import pytest
import torch

from actkv.kernels.compaction import apply_copies, plan_compaction
from actkv.kernels.lse_attn import action_scores
from actkv.paged import PagedKVCache, keep_mask_from_scores
from oracle import reference as ref

pytestmark = pytest.mark.gpu

BITS = {torch.float32: np.uint32, torch.float16: np.uint16, torch.bfloat16: np.uint16}


def _filled_cache(lens, bs=16, hkv=2, d=32, layers=1, seed=0, shuffle=True, dtype=torch.float32):
    """Same construction as the reference fixture (tests/test_kernels.py:19-30), on the GPU."""
    g = torch.Generator().manual_seed(seed)
    nb = sum(math.ceil(n / bs) for n in lens) + 8
    cache = PagedKVCache(nb, bs, hkv, d, n_layers=layers, dtype=dtype, device="cuda")
    if shuffle:
        cache.free = torch.randperm(nb, generator=g).tolist()
    for r, n in enumerate(lens):
        k = torch.randn(layers, n, hkv, d, generator=g).to(dtype)
        v = torch.randn(layers, n, hkv, d, generator=g).to(dtype)
        cache.append(r, k.cuda(), v.cuda())
    return cache


def _bits(t: torch.Tensor) -> np.ndarray:
    """Raw element bits of a tensor on the host (byte-exact comparisons)."""
    t = t.detach().cpu().contiguous()
    return t.view({4: torch.int32, 2: torch.int16, 1: torch.uint8}[t.element_size()]).numpy()


def _model_of(cache: PagedKVCache) -> ref.PagedCacheModel:
    """CPU oracle model holding the same bytes and allocator state as a GPU cache."""
    m = ref.PagedCacheModel(cache.num_blocks, cache.block_size, cache.n_kv_heads, cache.head_dim,
                            cache.n_layers, np_dtype=_bits(cache.kv[:1, :1, :1]).dtype)
    m.kv = _bits(cache.kv).copy()
    m.free = list(cache.free)
    m.tables = {r: list(t) for r, t in cache.tables.items()}
    m.seq_used = dict(cache.seq_used)
    return m


def _assert_same_state(cache, model):
    assert np.array_equal(_bits(cache.kv), model.kv), "KV bytes differ"
    assert cache.free == model.free
    assert cache.tables == model.tables
    assert cache.seq_used == model.seq_used


@pytest.mark.parametrize("lens,hq,hkv,d,bs,dtype", [
    ([37], 4, 2, 32, 16, torch.float32),
    ([5, 64, 100], 8, 2, 64, 16, torch.float32),
    ([33, 17], 6, 3, 24, 8, torch.float32),        # non-power-of-two head_dim and group size
    ([37, 300], 32, 8, 128, 16, torch.bfloat16),   # MFMA tile kernel, G = 4
    ([130, 19], 16, 8, 128, 16, torch.float16),    # MFMA, G = 2
    ([77], 8, 8, 128, 32, torch.bfloat16),         # MFMA, G = 1, block_size 32
])
def test_action_scores_matches_oracle(lens, hq, hkv, d, bs, dtype):
    cache = _filled_cache(lens, bs=bs, hkv=hkv, d=d, dtype=dtype)
    reqs = list(range(len(lens)))
    bt, seq = cache.block_table(reqs), cache.seq_tensor(reqs)
    width = bt.shape[1] * bs
    out_k = torch.zeros(len(reqs), hkv, width, device="cuda")
    n_k = torch.zeros(len(reqs), dtype=torch.int32, device="cuda")
    out_o = torch.zeros(len(reqs), hkv, width)
    n_o = torch.zeros(len(reqs), dtype=torch.int32)
    kv0 = cache.kv[0].cpu()
    tables = [cache.tables[r] for r in reqs]
    g = torch.Generator().manual_seed(1)
    for _ in range(3):  # three action tokens -> exercises the running mean
        q = torch.randn(len(reqs), hq, d, generator=g).to(dtype)
        lse = ref.decode_lse(q, kv0, tables, lens)
        action_scores(q.cuda(), cache.kv[0], bt, seq, lse.cuda(), out_k, n_k)
        ref.action_scores_fold(q, kv0, tables, lens, lse, out_o, n_o)
    rtol = 1e-4 if dtype == torch.float32 else 1e-3
    torch.testing.assert_close(out_k.cpu(), out_o, rtol=rtol, atol=1e-6)
    assert torch.equal(n_k.cpu(), n_o)


@pytest.mark.parametrize("hq,hkv,d,bs,qdt,kdt,n_q", [
    (6, 2, 24, 16, torch.float32, torch.float32, 50),      # G 3: 21 queries per chunk of 64 rows, 3 chunks
    (96, 1, 32, 16, torch.bfloat16, torch.bfloat16, 3),     # G 96 > 64 rows: head chunks 64 + 32, max carried
    (40, 1, 512, 16, torch.float16, torch.float16, 2),      # head dim 512: 16-row chunks, heads 16 + 16 + 8
    (16, 8, 256, 16, torch.bfloat16, torch.bfloat16, 20),   # head dim 256, G 2 (Gemma shape): 32-row chunks
    (32, 8, 128, 16, torch.float32, torch.bfloat16, 9),     # float32 queries on a bf16 cache
    (10, 2, 36, 12, torch.float16, torch.float16, 13),      # G 5, head dim 36, block 12
    (4, 2, 30, 16, torch.float32, torch.float32, 7),        # head dim 30 (not a multiple of 4): row-at-a-time kernel
])
def test_action_scores_generic_query_row_chunks(hq, hkv, d, bs, qdt, kdt, n_q):
    """The float32 path for shapes off the matrix cores walks the query rows (n, g) through LDS
    in chunks and keeps a chunk's dot products in registers: partial chunks, groups wider than
    a chunk (the max carried across head chunks), causal limits and partial query counts, against
    the oracle's folds."""
    lens = [300, 77]
    cache = _filled_cache(lens, bs=bs, hkv=hkv, d=d, dtype=kdt, seed=hq + d)
    reqs = list(range(len(lens)))
    bt, seq = cache.block_table(reqs), cache.seq_tensor(reqs)
    width = bt.shape[1] * bs
    kv0 = cache.kv[0].cpu()
    tables = [cache.tables[r] for r in reqs]
    g = torch.Generator().manual_seed(d + n_q)
    q = (torch.randn(len(reqs), n_q, hq, d, generator=g) * 0.5).to(qdt)
    lse = torch.stack([ref.decode_lse(q[:, n].float(), kv0, tables, lens) for n in range(n_q)], 1)
    n_valid = torch.tensor([n_q, max(1, n_q - 2)], dtype=torch.int32)
    kv_len = torch.stack([torch.randint(0, s + 3, (n_q,), generator=g) for s in lens]).to(torch.int32)
    out0 = torch.rand(len(reqs), hkv, width, generator=g)
    n0 = torch.tensor([2, 0], dtype=torch.int32)
    out_k, n_k = out0.cuda(), n0.cuda()
    action_scores(q.cuda(), cache.kv[0], bt, seq, lse.cuda(), out_k, n_k, n_valid=n_valid.cuda(), kv_len=kv_len.cuda())
    out_o, n_o = out0.clone(), n0.clone()
    ref.action_scores_nfold(q.float(), kv0, tables, lens, lse, out_o, n_o, n_valid=n_valid, kv_len=kv_len)
    rtol = 1e-4 if kdt == torch.float32 and qdt == torch.float32 else 1e-3
    torch.testing.assert_close(out_k.cpu(), out_o, rtol=rtol, atol=1e-6)
    assert torch.equal(n_k.cpu(), n_o)


@pytest.mark.parametrize("n_q,hq,hkv,dtype", [(37, 32, 8, torch.bfloat16), (129, 32, 8, torch.bfloat16),
                                              (40, 16, 8, torch.float16), (9, 6, 3, torch.float32),
                                              (300, 16, 8, torch.float16), (600, 8, 8, torch.bfloat16),
                                              # 320, 400 and 512 query rows: both MFMA kernels
                                              (80, 32, 8, torch.bfloat16), (100, 32, 8, torch.bfloat16),
                                              (128, 32, 8, torch.float16)])
def test_action_scores_n_queries_in_one_launch(n_q, hq, hkv, dtype):
    """N action tokens folded by one call == N reference folds (additive extension)."""
    lens = [200, 1000, 17]
    d = 128 if dtype != torch.float32 else 24
    cache = _filled_cache(lens, hkv=hkv, d=d, dtype=dtype, seed=3)
    reqs = list(range(len(lens)))
    bt, seq = cache.block_table(reqs), cache.seq_tensor(reqs)
    width = bt.shape[1] * 16
    g = torch.Generator().manual_seed(5)
    q = torch.randn(len(reqs), n_q, hq, d, generator=g).to(dtype)
    kv0 = cache.kv[0].cpu()
    tables = [cache.tables[r] for r in reqs]
    lse = torch.stack([ref.decode_lse(q[:, n], kv0, tables, lens) for n in range(n_q)], 1)
    out0 = torch.rand(len(reqs), hkv, width, generator=g)
    n0 = torch.tensor([0, 3, 1], dtype=torch.int32)
    out_k, n_k = out0.cuda(), n0.cuda()
    action_scores(q.cuda(), cache.kv[0], bt, seq, lse.cuda(), out_k, n_k)
    out_o, n_o = out0.clone(), n0.clone()
    ref.action_scores_nfold(q, kv0, tables, lens, lse, out_o, n_o)
    rtol = 1e-4 if dtype == torch.float32 else 1e-3
    torch.testing.assert_close(out_k.cpu(), out_o, rtol=rtol, atol=1e-6)
    assert torch.equal(n_k.cpu(), n_o)


def test_recovered_scores_are_probabilities():
    cache = _filled_cache([50], hkv=1, d=16)
    bt, seq = cache.block_table([0]), cache.seq_tensor([0])
    q = torch.randn(1, 1, 16)
    lse = ref.decode_lse(q, cache.kv[0].cpu(), [cache.tables[0]], [50])
    out = torch.zeros(1, 1, bt.shape[1] * 16, device="cuda")
    action_scores(q.cuda(), cache.kv[0], bt, seq, lse.cuda(), out, torch.zeros(1, dtype=torch.int32, device="cuda"))
    assert abs(float(out[0, 0, :50].sum()) - 1.0) < 1e-4
    assert float(out[0, 0, 50:].abs().sum()) == 0.0


def test_mfma_scores_are_probabilities():
    """Hq == Hkv (G = 1) on the bf16 MFMA path: each query's probabilities sum to 1."""
    cache = _filled_cache([1000], hkv=8, d=128, dtype=torch.bfloat16, seed=9)
    bt, seq = cache.block_table([0]), cache.seq_tensor([0])
    q = torch.randn(1, 8, 128).to(torch.bfloat16)
    lse = ref.decode_lse(q, cache.kv[0].cpu(), [cache.tables[0]], [1000])
    out = torch.zeros(1, 8, bt.shape[1] * 16, device="cuda")
    action_scores(q.cuda(), cache.kv[0], bt, seq, lse.cuda(), out, torch.zeros(1, dtype=torch.int32, device="cuda"))
    sums = out[0, :, :1000].sum(-1).cpu()
    torch.testing.assert_close(sums, torch.ones(8), rtol=0, atol=1e-4)
    assert float(out[0, :, 1000:].abs().sum()) == 0.0


@pytest.mark.parametrize("seq_used,budget,bs", [(100, 40, 16), (17, 10, 16), (64, 64, 16), (200, 3, 8),
                                                (5000, 1234, 16), (33, 0, 16)])
def test_plan_matches_oracle_and_is_conflict_free(seq_used, budget, bs):
    g = torch.Generator().manual_seed(seq_used)
    keep = torch.zeros(seq_used, dtype=torch.bool)
    keep[torch.randperm(seq_used, generator=g)[:budget]] = True
    table = torch.randperm(math.ceil(seq_used / bs) + 4, generator=g)
    plan = plan_compaction(keep.cuda(), seq_used, table.cuda(), bs)
    src_o, dst_o, perm_o, drop_o = ref.plan_compaction(keep.numpy(), seq_used, table.numpy(), bs)
    assert np.array_equal(plan.src_slots.cpu().numpy(), src_o)
    assert np.array_equal(plan.dst_slots.cpu().numpy(), dst_o)
    assert np.array_equal(plan.perm.cpu().numpy(), perm_o)
    assert plan.drop_blocks == drop_o
    src, dst = set(plan.src_slots.tolist()), set(plan.dst_slots.tolist())
    assert not (src & dst)
    assert sorted(plan.perm.tolist()) == sorted(torch.nonzero(keep).flatten().tolist())
    assert plan.drop_blocks == math.ceil(seq_used / bs) - math.ceil(budget / bs)


@pytest.mark.parametrize("dtype,planes,slots,row", [(torch.float32, 4, 300, 96), (torch.bfloat16, 6, 1000, 1024),
                                                    (torch.float16, 3, 77, 7), (torch.float32, 2, 50, 3)])
def test_copy_kernel_matches_oracle(dtype, planes, slots, row):
    g = torch.Generator().manual_seed(7)
    flat = torch.randn(planes, slots, row, generator=g).to(dtype)
    perm = torch.randperm(slots, generator=g)
    m = slots // 3
    src, dst = perm[:m], perm[m:2 * m]
    a = flat.cuda()
    apply_copies(a, src.cuda(), dst.cuda())
    b = _bits(flat).copy()
    ref.apply_copies(b, src.numpy(), dst.numpy())
    assert np.array_equal(_bits(a), b)


def test_copy_kernel_handles_offsets_past_2_to_the_31():
    """Multi-layer caches put later planes past 2^31 elements; int32 offsets would wrap there."""
    row = 1024
    slots = 2**31 // row // 2 + 64                      # each plane holds just over 2^30 elements
    flat = torch.zeros(3, slots, row, dtype=torch.float16, device="cuda")
    src = torch.tensor([5, slots - 1], device="cuda")
    dst = torch.tensor([7, 9], device="cuda")
    flat[:, src] = torch.arange(1, 4, dtype=torch.float16, device="cuda").view(3, 1, 1)
    apply_copies(flat, src, dst)
    torch.cuda.synchronize()
    assert torch.equal(flat[:, dst], flat[:, src])
    del flat
    torch.cuda.empty_cache()


@pytest.mark.parametrize("n,budget,dtype", [(150, 60, torch.float32), (40, 39, torch.float32), (33, 16, torch.float32),
                                            (1000, 101, torch.bfloat16), (2048, 2047, torch.float16)])
def test_compaction_is_bit_exact_and_frees_blocks(n, budget, dtype):
    cache = _filled_cache([n], layers=2, dtype=dtype)
    model = _model_of(cache)
    k_before = [cache.gather(0, layer)[0].clone() for layer in range(2)]
    used_before = cache.used_blocks
    keep = torch.zeros(n, dtype=torch.bool)
    keep[torch.randperm(n, generator=torch.Generator().manual_seed(n))[:budget]] = True
    perm = cache.compact(0, keep.cuda())
    perm_o = model.compact(0, keep.numpy())
    assert np.array_equal(perm.cpu().numpy(), perm_o)
    _assert_same_state(cache, model)
    assert cache.seq_used[0] == budget
    for layer in range(2):
        assert torch.equal(cache.gather(0, layer)[0], k_before[layer][perm])
    assert used_before - cache.used_blocks == math.ceil(n / 16) - math.ceil(budget / 16)


def test_attention_is_invariant_to_compaction_permutation():
    cache = _filled_cache([90], hkv=2, d=32)
    keep = torch.zeros(90, dtype=torch.bool, device="cuda")
    keep[torch.randperm(90)[:41].cuda()] = True
    k, v = cache.gather(0)
    k_kept, v_kept = k[keep], v[keep]
    q = torch.randn(1, 4, 32, device="cuda")
    other = _filled_cache([1], hkv=2, d=32)
    other.release(0)
    other.append(0, k_kept.unsqueeze(0), v_kept.unsqueeze(0))
    want, _ = other.decode_attention([0], q)
    cache.compact(0, keep)
    got, _ = cache.decode_attention([0], q)
    torch.testing.assert_close(got, want, rtol=1e-4, atol=1e-5)


def test_evict_keeps_the_protected_prefix_and_the_top_scored_tokens():
    cache = _filled_cache([70], hkv=2, d=16, layers=2)
    model = _model_of(cache)
    k_before, v_before = cache.gather(0, layer=1)
    scores = 0.1 * torch.rand(2, 2, 70, generator=torch.Generator().manual_seed(3))
    hot = [5, 17, 40, 69]
    scores[..., hot] += 1.0
    perm = cache.evict(0, scores.cuda(), budget=4, protected=3)
    assert sorted(perm.tolist()) == [0, 1, 2, *hot]
    k_after, v_after = cache.gather(0, layer=1)
    assert torch.equal(k_after, k_before[perm])
    assert torch.equal(v_after, v_before[perm])
    assert cache.seq_used[0] == 7 and len(cache.tables[0]) == 1
    perm_o = model.evict(0, scores, budget=4, protected=3)
    assert np.array_equal(perm.cpu().numpy(), perm_o)
    _assert_same_state(cache, model)
    assert np.array_equal(cache.pinned[0].cpu().numpy(), model.pinned[0])


def test_evictions_on_two_side_streams_match_the_oracle():
    """Evictions with equal budgets on two side streams (ordered by a stream wait, as calls that
    share the keep-mask workspace must be): the budget and table uploads of one stream are not
    read by the other stream's kernels, and the final state equals the oracle's."""
    cache = _filled_cache([300, 500, 260], hkv=2, d=16, seed=41)
    model = _model_of(cache)
    g = torch.Generator().manual_seed(42)
    sc = [torch.rand(2, n, generator=g) for n in (300, 500, 260)]
    dev_sc = [s.cuda() for s in sc]
    torch.cuda.synchronize()
    a, b = torch.cuda.Stream(), torch.cuda.Stream()
    perms = []
    with torch.cuda.stream(a):
        perms.append(cache.evict(0, dev_sc[0], budget=100, protected=4))
    b.wait_stream(a)
    with torch.cuda.stream(b):
        perms.append(cache.evict(1, dev_sc[1], budget=100, protected=4))
    a.wait_stream(b)
    with torch.cuda.stream(a):
        perms.append(cache.evict(2, dev_sc[2], budget=100, protected=4))
    torch.cuda.synchronize()
    for r in range(3):
        want = model.evict(r, sc[r], budget=100, protected=4)
        assert np.array_equal(perms[r].cpu().numpy(), want)
    _assert_same_state(cache, model)


@pytest.mark.parametrize("offset,any_byte", [(0, False), (1, False), (16, False), (0, True), (1, True)])
def test_pack_keep_matches_numpy(offset, any_byte):
    """actkv_pack_keep (keep mask bytes -> LSB-first bits, zero to whole blocks, kept counts) on
    rows that are 16-byte aligned (offset 0, 16) or not (offset 1): the vector and byte paths.
    A kept byte is 1, or (any_byte, through the C ABI) any nonzero value 1..255: both paths
    keep every nonzero byte."""
    from actkv import _hip
    g = torch.Generator().manual_seed(offset + 100 * any_byte)
    lens, bs = [70001, 33, 65, 4096], 16
    R, W = len(lens), 70016 + 48
    full = torch.rand(R, W + offset, generator=g) < 0.3
    if any_byte:
        full = full.to(torch.uint8) * torch.randint(1, 256, full.shape, generator=g, dtype=torch.uint8)
        assert (full == 128).any() and (full == 255).any() and (full == 1).any()
    keep_cpu = full[:, offset:offset + W] != 0
    keep = full.cuda()[:, offset:offset + W]
    seq = torch.tensor(lens, dtype=torch.int32, device="cuda")
    nw = (-(-max(lens) // bs) * bs + 31) // 32
    bits = torch.full((R, nw), -1, dtype=torch.int32, device="cuda")
    kept = torch.full((R,), -1, dtype=torch.int32, device="cuda")
    rc = _hip.lib().actkv_pack_keep(keep.data_ptr(), keep.stride(0), R, seq.data_ptr(), bs, bits.data_ptr(),
                                    bits.stride(0), kept.data_ptr(), max(lens), _hip.stream(keep.device))
    assert rc == 0
    got = bits.cpu().numpy().view(np.uint32)
    for r, S in enumerate(lens):
        padded = -(-S // bs) * bs
        want = np.zeros(padded, dtype=bool)
        want[:S] = keep_cpu[r, :S].numpy()
        words = np.packbits(np.pad(want, (0, (-padded) % 32)).reshape(-1, 32)[:, ::-1], axis=1, bitorder="big")
        want_w = words.view(">u4").reshape(-1).astype(np.uint32)
        assert np.array_equal(got[r, :want_w.size], want_w), f"row {r}: bits differ"
        assert int(kept[r]) == int(keep_cpu[r, :S].sum())


def test_evict_within_budget_is_a_no_op():
    cache = _filled_cache([20])
    table = list(cache.tables[0])
    assert cache.evict(0, torch.rand(2, 20, device="cuda"), budget=20).tolist() == list(range(20))
    assert cache.tables[0] == table and cache.seq_used[0] == 20


def test_keep_mask_reduces_heads_then_averages_layers():
    scores = torch.zeros(2, 2, 4)
    scores[0, 0, 1] = 1.0
    scores[:, :, 2] = 0.3
    assert keep_mask_from_scores(scores.cuda(), 4, budget=1).tolist() == [False, False, True, False]
    assert keep_mask_from_scores(scores.cuda(), 4, budget=1, head_reduce="max").tolist() == [False, True, False, False]


def test_evict_keeps_the_protected_tokens_across_repeated_evictions():
    cache = _filled_cache([64], hkv=2, d=16)
    model = _model_of(cache)
    prompt = cache.gather(0)[0][:8].clone()
    scores = torch.zeros(2, 64)
    scores[:, 8:56] = torch.rand(2, 48, generator=torch.Generator().manual_seed(4)) + 1
    cache.evict(0, scores.cuda(), budget=24, protected=8)
    model.evict(0, scores, budget=24, protected=8)
    new = torch.randn(1, 16, 2, 16, generator=torch.Generator().manual_seed(5))
    cache.append(0, new.cuda(), new.cuda())
    model.append(0, _bits(new), _bits(new))
    scores = torch.zeros(2, cache.seq_used[0])
    scores[:, -16:] = 1.0
    perm = cache.evict(0, scores.cuda(), budget=16, protected=8)
    perm_o = model.evict(0, scores, budget=16, protected=8)
    k = cache.gather(0)[0]
    assert cache.seq_used[0] == 8 + 16
    assert all(any(torch.equal(p, row) for row in k) for p in prompt)
    assert np.array_equal(np.sort(perm.cpu().numpy()), np.sort(perm_o))
    _assert_same_state(cache, model)


@pytest.mark.parametrize("dtype,hq,hkv,d,bs,n_q", [
    (torch.bfloat16, 32, 8, 128, 16, 23), (torch.float16, 16, 8, 128, 32, 23),
    (torch.bfloat16, 8, 8, 128, 16, 23), (torch.float32, 6, 3, 24, 8, 23),
    # query tiles of 385..512 rows (query tile in registers) and 257..384 rows (K slices)
    (torch.bfloat16, 32, 8, 128, 16, 100), (torch.float16, 16, 8, 128, 16, 150),
    (torch.bfloat16, 8, 8, 128, 16, 300), (torch.float16, 32, 8, 128, 16, 128),
    (torch.bfloat16, 16, 8, 128, 64, 200),
    # G = 1 with 400 query rows: the query-register kernel's per-row causal limits
    (torch.bfloat16, 8, 8, 128, 16, 400)])
def test_action_scores_causal_region_and_ragged_query_counts(dtype, hq, hkv, d, bs, n_q):
    """kv_len (query n sees tokens t < kv_len[r, n]) and n_valid (request r folds its first
    n_valid[r] queries): the causal action region of an agent round (additive extension)."""
    lens = [700, 90, 1500]
    cache = _filled_cache(lens, bs=bs, hkv=hkv, d=d, dtype=dtype, seed=11)
    reqs = list(range(len(lens)))
    bt, seq = cache.block_table(reqs), cache.seq_tensor(reqs)
    width = bt.shape[1] * bs
    g = torch.Generator().manual_seed(12)
    q = torch.randn(len(reqs), n_q, hq, d, generator=g).to(dtype)
    kv0 = cache.kv[0].cpu()
    tables = [cache.tables[r] for r in reqs]
    lse = torch.stack([ref.decode_lse(q[:, n], kv0, tables, lens) for n in range(n_q)], 1)
    n_valid = torch.tensor([n_q, 5, 17], dtype=torch.int32)
    kv_len = torch.stack([torch.randint(1, s + 1, (n_q,), generator=g) for s in lens]).to(torch.int32)
    kv_len[0, 3] = lens[0]
    out0 = torch.rand(len(reqs), hkv, width, generator=g)
    n0 = torch.tensor([2, 0, 7], dtype=torch.int32)
    out_k, n_k = out0.cuda(), n0.cuda()
    action_scores(q.cuda(), cache.kv[0], bt, seq, lse.cuda(), out_k, n_k, n_valid=n_valid.cuda(), kv_len=kv_len.cuda())
    out_o, n_o = out0.clone(), n0.clone()
    ref.action_scores_nfold(q, kv0, tables, lens, lse, out_o, n_o, n_valid=n_valid, kv_len=kv_len)
    rtol = 1e-4 if dtype == torch.float32 else 1e-3
    torch.testing.assert_close(out_k.cpu(), out_o, rtol=rtol, atol=1e-6)
    assert torch.equal(n_k.cpu(), n_o)


@pytest.mark.parametrize("dtype,hq,hkv,d,n_q", [
    (torch.float32, 8, 2, 32, 5),            # generic kernel
    (torch.bfloat16, 32, 8, 128, 80),        # 320 query rows: K-slice kernel
    (torch.bfloat16, 32, 8, 128, 100),       # 400 query rows: query-register kernel
    (torch.float16, 16, 8, 128, 24),         # 48 rows, causal below
])
def test_action_scores_leave_tokens_of_out_of_pool_blocks_untouched(dtype, hq, hkv, d, n_q):
    """A block-table entry outside [0, num_blocks) inside seq_used: every kernel reads in bounds
    and leaves that block's score columns as they were; every other column is scored."""
    lens = [600, 333]
    bs = 16
    cache = _filled_cache(lens, bs=bs, hkv=hkv, d=d, dtype=dtype, seed=21)
    reqs = [0, 1]
    bt, seq = cache.block_table(reqs), cache.seq_tensor(reqs)
    width = bt.shape[1] * bs
    g = torch.Generator().manual_seed(22)
    q = torch.randn(2, n_q, hq, d, generator=g).to(dtype)
    kv0 = cache.kv[0].cpu()
    tables = [cache.tables[r] for r in reqs]
    lse = torch.stack([ref.decode_lse(q[:, n], kv0, tables, lens) for n in range(n_q)], 1)
    out0 = torch.rand(2, hkv, width, generator=g)
    kv_len = None
    if n_q == 24:
        kv_len = torch.stack([torch.randint(1, s + 1, (n_q,), generator=g) for s in lens]).to(torch.int32)
    bad = bt.clone()
    bad[0, 3] = -1                       # tokens 48..63 of request 0
    bad[1, 10] = cache.num_blocks + 7    # tokens 160..175 of request 1
    out_k = out0.cuda()
    action_scores(q.cuda(), cache.kv[0], bad, seq, lse.cuda(), out_k,
                  torch.zeros(2, dtype=torch.int32, device="cuda"),
                  kv_len=None if kv_len is None else kv_len.cuda())
    out_o = out0.clone()
    ref.action_scores_nfold(q, kv0, tables, lens, lse, out_o, torch.zeros(2, dtype=torch.int32), kv_len=kv_len)
    got = out_k.cpu()
    untouched = torch.zeros(2, width, dtype=torch.bool)
    untouched[0, 48:64] = True
    untouched[1, 160:176] = True
    for r in range(2):
        assert torch.equal(got[r][:, untouched[r]], out0[r][:, untouched[r]])
        keep = ~untouched[r]
        rtol = 1e-4 if dtype == torch.float32 else 1e-3
        torch.testing.assert_close(got[r][:, keep], out_o[r][:, keep], rtol=rtol, atol=1e-6)


@pytest.mark.parametrize("hq,hkv,n_q,half,d", [
    (32, 8, 16, 0, 128),      # 64 rows: 8 KV heads per workgroup
    (32, 8, 32, 1, 128),      # 128 rows: 4 KV heads per workgroup
    (8, 8, 9, 1, 128),        # group 1, 9 rows: 8 heads per workgroup
    (16, 4, 30, 0, 128),      # group 4 over 4 KV heads, 120 rows: 4 heads per workgroup
    (32, 8, 16, 1, 64),       # head dim 64, 64 rows: 8 KV heads per workgroup
    (8, 8, 9, 0, 64),         # head dim 64, group 1, 9 rows
])
def test_action_scores_heads_per_workgroup_with_strided_heads(hq, hkv, n_q, half, d):
    """Small query tiles score several KV heads of the same tokens in one workgroup, reading
    each token's heads side by side.  K here is a view with a head stride of 2 x head_dim
    (every other head_dim-element piece of a wider row, starting at piece `half`), so the
    heads are not contiguous; with ragged query counts, causal limits and two out-of-pool
    table entries, against the oracle's folds."""
    bs, lens = 16, [700, 333, 1400]
    R = len(lens)
    g = torch.Generator().manual_seed(40 + n_q)
    nb = sum(-(-s // bs) for s in lens) + 5
    wide = torch.randn(2, nb, bs, hkv, 2 * d, generator=g).to(torch.bfloat16)
    kv = wide.cuda()[..., half * d:(half + 1) * d]
    assert kv.stride(-2) == 2 * d and not kv.is_contiguous()
    perm = torch.randperm(nb, generator=g).tolist()
    tables, pos = [], 0
    for s in lens:
        nblk = -(-s // bs)
        tables.append(perm[pos:pos + nblk])
        pos += nblk
    mb = max(len(t) for t in tables)
    bt = torch.zeros(R, mb, dtype=torch.int32)
    for r, t in enumerate(tables):
        bt[r, :len(t)] = torch.tensor(t, dtype=torch.int32)
    kv0 = wide[..., half * d:(half + 1) * d].contiguous()
    q = torch.randn(R, n_q, hq, d, generator=g).to(torch.bfloat16)
    lse = torch.stack([ref.decode_lse(q[:, n], kv0, tables, lens) for n in range(n_q)], 1)
    n_valid = torch.tensor([n_q, max(1, n_q // 3), n_q - 1], dtype=torch.int32)
    kv_len = torch.stack([torch.randint(1, s + 1, (n_q,), generator=g) for s in lens]).to(torch.int32)
    width = mb * bs
    out0 = torch.rand(R, hkv, width, generator=g)
    n0 = torch.tensor([3, 0, 1], dtype=torch.int32)
    bad = bt.clone()
    bad[0, 5] = -1                      # tokens 80..95 of request 0
    bad[2, 40] = nb + 3                 # tokens 640..655 of request 2
    out_k, n_k = out0.cuda(), n0.cuda()
    action_scores(q.cuda(), kv, bad.cuda(), torch.tensor(lens, dtype=torch.int32, device="cuda"), lse.cuda(),
                  out_k, n_k, n_valid=n_valid.cuda(), kv_len=kv_len.cuda())
    out_o, n_o = out0.clone(), n0.clone()
    ref.action_scores_nfold(q, kv0, tables, lens, lse, out_o, n_o, n_valid=n_valid, kv_len=kv_len)
    got = out_k.cpu()
    untouched = torch.zeros(R, width, dtype=torch.bool)
    untouched[0, 80:96] = True
    untouched[2, 640:656] = True
    for r in range(R):
        assert torch.equal(got[r][:, untouched[r]], out0[r][:, untouched[r]]), f"request {r}: out-of-pool columns"
        keep = ~untouched[r]
        torch.testing.assert_close(got[r][:, keep], out_o[r][:, keep], rtol=1e-3, atol=1e-6)
    assert torch.equal(n_k.cpu(), n_o)


@pytest.mark.parametrize("hq,hkv,n_q,dtype", [
    (32, 8, 16, torch.bfloat16),    # 64 rows: 8 KV heads per workgroup
    (32, 8, 32, torch.float16),     # 128 rows: 4 KV heads per workgroup
    (6, 3, 40, torch.bfloat16),     # 80 rows over 3 KV heads: one head, 2 row groups
    (32, 8, 60, torch.bfloat16),    # 240 rows: K-slice kernel
    (32, 8, 100, torch.bfloat16),   # 400 rows: query tile in registers, 8 row groups
])
def test_action_scores_ragged_lengths_in_a_padded_table(hq, hkv, n_q, dtype):
    """Requests of very different lengths in a block table padded well past the longest: the
    launch is sized for the table, so most of a short request's token ranges are empty and
    each pair takes its ranges in rotated order.  Every token below seq_used is scored as the
    oracle scores it; every column past it (whose padded entries name a valid block) is left
    as it was."""
    lens = [2900, 45, 1333, 700]
    bs, d = 16, 128
    cache = _filled_cache(lens, bs=bs, hkv=hkv, d=d, dtype=dtype, seed=31)
    reqs = list(range(len(lens)))
    bt0, seq = cache.block_table(reqs), cache.seq_tensor(reqs)
    pad = 150
    bt = torch.zeros(len(reqs), bt0.shape[1] + pad, dtype=torch.int32, device="cuda")
    bt[:, :bt0.shape[1]] = bt0
    width = bt.shape[1] * bs
    g = torch.Generator().manual_seed(32)
    q = torch.randn(len(reqs), n_q, hq, d, generator=g).to(dtype)
    kv0 = cache.kv[0].cpu()
    tables = [cache.tables[r] for r in reqs]
    lse = torch.stack([ref.decode_lse(q[:, n], kv0, tables, lens) for n in range(n_q)], 1)
    out0 = torch.rand(len(reqs), hkv, width, generator=g)
    n0 = torch.tensor([0, 2, 5, 1], dtype=torch.int32)
    out_k, n_k = out0.cuda(), n0.cuda()
    action_scores(q.cuda(), cache.kv[0], bt, seq, lse.cuda(), out_k, n_k)
    out_o, n_o = out0.clone(), n0.clone()
    ref.action_scores_nfold(q, kv0, tables, lens, lse, out_o, n_o)
    got = out_k.cpu()
    for r, s in enumerate(lens):
        torch.testing.assert_close(got[r][:, :s], out_o[r][:, :s], rtol=1e-3, atol=1e-6)
        assert torch.equal(got[r][:, s:], out0[r][:, s:])
    assert torch.equal(n_k.cpu(), n_o)


@pytest.mark.parametrize("dtype,hq,hkv,n_q,causal,partial", [
    (torch.bfloat16, 64, 8, 5, False, False),    # 40 rows: 2 row groups
    (torch.bfloat16, 64, 8, 24, True, True),     # 192 rows: 4 row groups, causal, partial counts
    (torch.float16, 16, 2, 64, False, True),     # 512 rows: 8 row groups, fragment layout
    (torch.bfloat16, 64, 8, 64, True, False),    # 512 rows, causal
    (torch.bfloat16, 16, 2, 100, True, True),    # 800 rows: two launches (64 + 36 queries)
    (torch.float16, 64, 8, 16, True, False),     # 128 rows, causal
    (torch.bfloat16, 24, 8, 12, True, False),    # G = 3 padded to 4: 48 rows, 8 heads per workgroup
    (torch.bfloat16, 24, 8, 90, False, True),    # G = 3: 360 rows
    (torch.float16, 40, 8, 30, True, True),      # G = 5 padded to 8: 240 rows
    (torch.bfloat16, 48, 8, 70, True, False),    # G = 6: two launches (64 + 6 queries)
    (torch.bfloat16, 28, 4, 9, False, False),    # G = 7: 72 rows
    (torch.bfloat16, 128, 8, 10, True, True),    # G = 16 (Llama-3.1-405B): 160 rows
    (torch.float16, 128, 8, 32, False, False),   # G = 16: 512 rows
    (torch.bfloat16, 32, 2, 70, True, False),    # G = 16: three launches (32 + 32 + 6 queries)
    (torch.bfloat16, 96, 8, 40, True, True),     # G = 12 padded to 16: two launches
    (torch.float16, 72, 8, 7, False, False),     # G = 9 padded to 16: 112 rows
])
def test_action_scores_groups_of_eight_heads(dtype, hq, hkv, n_q, causal, partial):
    """G = 8 (64 query heads over 8 KV heads, as Qwen3-32B): a query's eight heads span both
    halves of a wave, and the max over them is taken across the halves before the exp.  Groups
    of 3, 5, 6 and 7 are laid out as 4 or 8 rows per query with padding rows that never win
    the max."""
    lens = [700, 90, 1500]
    d, bs = 128, 16
    cache = _filled_cache(lens, bs=bs, hkv=hkv, d=d, dtype=dtype, seed=41)
    reqs = list(range(len(lens)))
    bt, seq = cache.block_table(reqs), cache.seq_tensor(reqs)
    width = bt.shape[1] * bs
    g = torch.Generator().manual_seed(42)
    q = torch.randn(len(reqs), n_q, hq, d, generator=g).to(dtype)
    kv0 = cache.kv[0].cpu()
    tables = [cache.tables[r] for r in reqs]
    lse = torch.stack([ref.decode_lse(q[:, n], kv0, tables, lens) for n in range(n_q)], 1)
    n_valid = torch.tensor([n_q, min(3, n_q), max(n_q - 7, 0)], dtype=torch.int32) if partial else None
    kv_len = None
    if causal:
        kv_len = torch.stack([torch.randint(1, s + 1, (n_q,), generator=g) for s in lens]).to(torch.int32)
        kv_len[0, 0] = lens[0]
    out0 = torch.rand(len(reqs), hkv, width, generator=g)
    n0 = torch.tensor([1, 0, 4], dtype=torch.int32)
    out_k, n_k = out0.cuda(), n0.cuda()
    action_scores(q.cuda(), cache.kv[0], bt, seq, lse.cuda(), out_k, n_k,
                  n_valid=None if n_valid is None else n_valid.cuda(),
                  kv_len=None if kv_len is None else kv_len.cuda())
    out_o, n_o = out0.clone(), n0.clone()
    ref.action_scores_nfold(q, kv0, tables, lens, lse, out_o, n_o, n_valid=n_valid, kv_len=kv_len)
    torch.testing.assert_close(out_k.cpu(), out_o, rtol=1e-3, atol=1e-6)
    assert torch.equal(n_k.cpu(), n_o)


@pytest.mark.parametrize("dtype,hq,hkv,n_q,causal,partial", [
    (torch.bfloat16, 64, 8, 10, True, True),     # GPT-OSS shape (G = 8): 80 rows
    (torch.bfloat16, 64, 8, 64, False, False),   # G = 8: 512 rows
    (torch.float16, 32, 8, 100, True, False),    # G = 4: 400 rows, fragment layout
    (torch.bfloat16, 32, 8, 12, False, True),    # G = 4: 48 rows, 8 heads per workgroup
    (torch.bfloat16, 32, 8, 30, True, False),    # G = 4: 120 rows, 4 heads per workgroup
    (torch.float16, 16, 8, 70, False, False),    # G = 2: 140 rows
    (torch.bfloat16, 8, 8, 300, True, True),     # G = 1: 300 rows
    (torch.bfloat16, 128, 8, 40, True, False),   # G = 16: two launches
])
def test_action_scores_head_dim_64(dtype, hq, hkv, n_q, causal, partial):
    """head_dim 64 (GPT-OSS, Llama-3.2-1B): the query-register kernel with 128-byte head pieces
    (4 k steps, 8 swizzled 16-byte columns)."""
    lens = [700, 90, 1500]
    d, bs = 64, 16
    cache = _filled_cache(lens, bs=bs, hkv=hkv, d=d, dtype=dtype, seed=51)
    reqs = list(range(len(lens)))
    bt, seq = cache.block_table(reqs), cache.seq_tensor(reqs)
    width = bt.shape[1] * bs
    g = torch.Generator().manual_seed(52)
    q = torch.randn(len(reqs), n_q, hq, d, generator=g).to(dtype)
    kv0 = cache.kv[0].cpu()
    tables = [cache.tables[r] for r in reqs]
    lse = torch.stack([ref.decode_lse(q[:, n], kv0, tables, lens) for n in range(n_q)], 1)
    n_valid = torch.tensor([n_q, min(3, n_q), max(n_q - 7, 0)], dtype=torch.int32) if partial else None
    kv_len = None
    if causal:
        kv_len = torch.stack([torch.randint(1, s + 1, (n_q,), generator=g) for s in lens]).to(torch.int32)
        kv_len[0, 0] = lens[0]
    out0 = torch.rand(len(reqs), hkv, width, generator=g)
    n0 = torch.tensor([1, 0, 4], dtype=torch.int32)
    out_k, n_k = out0.cuda(), n0.cuda()
    action_scores(q.cuda(), cache.kv[0], bt, seq, lse.cuda(), out_k, n_k,
                  n_valid=None if n_valid is None else n_valid.cuda(),
                  kv_len=None if kv_len is None else kv_len.cuda())
    out_o, n_o = out0.clone(), n0.clone()
    ref.action_scores_nfold(q, kv0, tables, lens, lse, out_o, n_o, n_valid=n_valid, kv_len=kv_len)
    torch.testing.assert_close(out_k.cpu(), out_o, rtol=1e-3, atol=1e-6)
    assert torch.equal(n_k.cpu(), n_o)


def test_action_scores_every_layer_in_one_launch():
    """kv [L, 2, ...] with q [L, R, N, Hq, D]: each layer scored against its own K (extension)."""
    lens = [300, 77]
    L, hq, hkv, d, n_q = 3, 32, 8, 128, 6
    cache = _filled_cache(lens, hkv=hkv, d=d, layers=L, dtype=torch.bfloat16, seed=13)
    reqs = [0, 1]
    width = cache.block_table(reqs).shape[1] * 16
    g = torch.Generator().manual_seed(14)
    q = torch.randn(L, 2, n_q, hq, d, generator=g).to(torch.bfloat16)
    tables = [cache.tables[r] for r in reqs]
    kvs = [cache.kv[l].cpu() for l in range(L)]
    lse = torch.stack([torch.stack([ref.decode_lse(q[l, :, n], kvs[l], tables, lens) for n in range(n_q)], 1)
                       for l in range(L)])
    out = torch.zeros(L, 2, hkv, width, device="cuda")
    n_seen = torch.zeros(2, dtype=torch.int32, device="cuda")
    cache.cal_attn(reqs, q.cuda(), lse.cuda(), out, n_seen, layer=None)
    for l in range(L):
        want = torch.zeros(2, hkv, width)
        ref.action_scores_nfold(q[l], kvs[l], tables, lens, lse[l], want, torch.zeros(2, dtype=torch.int32))
        torch.testing.assert_close(out[l].cpu(), want, rtol=1e-3, atol=1e-6)
    assert n_seen.tolist() == [n_q, n_q]


@pytest.mark.parametrize("L,H,S,W,budget,prot,reduce", [
    (36, 8, 4096, 4096, 409, 4, "mean"),     # Qwen3-8B layer/head counts
    (36, 8, 3001, 3072, 300, 0, "mean"),     # S not a multiple of 32: torch's tail-column order
    (20, 8, 1000, 1024, 100, 7, "max"),
    (1, 8, 777, 800, 77, 4, "mean"),
    (3, 3, 200, 200, 20, 0, "mean"),
    (40, 16, 513, 520, 64, 2, "mean"),       # 16 heads: a full cascade block per layer
    (5, 8, 1001, 1001, 99, 3, "mean"),       # rows not 16-byte aligned: the 4-byte load path
    (2, 4, 2050, 2052, 200, 0, "max"),       # 4 heads, a last quad with 2 tokens
    # more than 120 layers: 64-token key blocks
    (121, 8, 1500, 1504, 150, 4, "mean"),
    (256, 2, 700, 704, 70, 0, "max"),
    (200, 3, 333, 333, 33, 2, "mean"),       # unaligned rows: the one-element load path
])
def test_keep_mask_bit_exact_with_the_oracle(L, H, S, W, budget, prot, reduce):
    """The device reduction reproduces torch's CPU mean bit for bit, so the keep mask equals
    the oracle's on the same scores (distinct scores: no top-k ties)."""
    g = torch.Generator().manual_seed(L * 1000 + S)
    scores = torch.rand(L, H, W, generator=g) * torch.exp(torch.randn(L, H, W, generator=g))
    want = ref.keep_mask_from_scores(scores, S, budget, protected=prot, head_reduce=reduce)
    got = keep_mask_from_scores(scores.cuda(), S, budget, protected=prot, head_reduce=reduce).cpu()
    assert torch.equal(got, want)
    assert int(got.sum()) == min(prot, S) + budget


@pytest.mark.parametrize("dtype,reduce,prot_kind", [
    (torch.float32, "mean", "count"),
    (torch.float32, "max", "mask"),
    (torch.bfloat16, "mean", "mask"),
])
def test_keep_mask_ragged_batch_in_one_call_matches_the_oracle(dtype, reduce, prot_kind):
    """One keep-mask call over ragged requests -- past the selection's 32768-token register
    chunk, exactly one chunk, a few blocks, a few tokens -- equals the oracle request by
    request: the bool mask, and the packed bits (LSB-first, zero up to whole blocks)."""
    from actkv import _hip
    from actkv.paged import _keep_mask_launch
    lens = [70001, 13103, 5, 40000, 1, 32768, 257]
    budgets = [7000, 1027, 2, 0, 1, 3276, 300]
    L, H, R, bs = 4, 8, len(lens), 16
    W = max(lens) + 3
    g = torch.Generator().manual_seed(31)
    scores = (torch.rand(L, R, H, W, generator=g) * torch.exp(torch.randn(L, R, H, W, generator=g))).to(dtype)
    dev = torch.device("cuda")
    sc = scores.to(dev)
    seq = _hip.upload_i32(lens, dev)
    bud = _hip.upload_i32(budgets, dev)
    if prot_kind == "count":
        prots = [4, 0, 2, 9, 0, 4, 300]
        pc, pm = _hip.upload_i32(prots, dev), None
        pm_cpu = [torch.arange(s) < p for s, p in zip(lens, prots)]
    else:
        pm_full = torch.rand(R, W, generator=g) < 0.03
        pc, pm = None, pm_full.to(dev)
        pm_cpu = [pm_full[r, :s] for r, s in enumerate(lens)]
    keep, bits = _keep_mask_launch(sc, L, H, sc.stride(0), sc.stride(1), sc.stride(2), R, seq, bud, pc, pm,
                                   0 if pm is None else pm.stride(0), reduce, bs, max(lens), dev)
    keep, bits = keep.cpu(), bits.cpu().numpy().view(np.uint32)
    for r, S in enumerate(lens):
        want = ref.keep_mask_from_scores(scores[:, r].float(), S, budgets[r], protected=pm_cpu[r], head_reduce=reduce)
        assert torch.equal(keep[r, :S], want), f"request {r} ({S} tokens): keep mask differs"
        padded = -(-S // bs) * bs
        unpacked = np.unpackbits(bits[r].view(np.uint8), bitorder="little")[:padded].astype(bool)
        assert np.array_equal(unpacked[:S], want.numpy()) and not unpacked[S:].any(), f"request {r}: keep bits"


def test_keep_mask_ties_keep_the_lower_index():
    """Equal scores straddling the top-k boundary: the lower index wins (documented rule)."""
    S = 5000
    scores = torch.zeros(2, 4, S)
    scores[..., 100:1100] = 0.5                      # 1000 tied candidates, 300 of them kept
    scores[..., 3000:3050] = 1.0                     # 50 strictly higher
    keep = keep_mask_from_scores(scores.cuda(), S, 350, protected=3).cpu()
    want = ref.keep_mask_lowest_index_ties(scores, S, 350, protected=3)
    assert torch.equal(keep, want)
    assert keep[:3].all() and keep[3000:3050].all() and keep[100:400].all() and not keep[400:1100].any()


@pytest.mark.parametrize("n_tied,spread,S", [(5000, True, 40000), (3000, False, 40000), (40, True, 40000),
                                             (5000, True, 30000), (40, True, 30000)])
def test_keep_mask_many_ties_keep_the_lower_index(n_tied, spread, S):
    """More tied scores at the boundary than the selection ranks in LDS (2048), scattered over
    the request or in one run, and a few ties among distinct scores: lowest indices first.
    40000 tokens exceed the select block's LDS chunk of keys (candidates gathered), 30000 do not
    (ties found among the keys in LDS)."""
    g = torch.Generator().manual_seed(n_tied)
    scores = torch.rand(3, 2, S, generator=g) * 0.4            # distinct, below the tie value
    pos = torch.randperm(S - 8, generator=g)[:n_tied] + 8 if spread else torch.arange(1000, 1000 + n_tied)
    scores[..., pos] = 0.5
    scores[..., S - 100:] = 0.9                                # 100 strictly higher
    budget = 100 + n_tied // 3
    keep = keep_mask_from_scores(scores.cuda(), S, budget, protected=4).cpu()
    want = ref.keep_mask_lowest_index_ties(scores, S, budget, protected=4)
    assert torch.equal(keep, want)
    assert int(keep.sum()) == 4 + budget


def test_batched_evict_mixes_first_and_repeated_evictions():
    """evict_batch over requests whose pins are a prefix count (first eviction) and requests
    that carry a pinned mask from an earlier eviction equals sequential oracle evicts."""
    cache = _filled_cache([90, 120, 75], hkv=2, d=16, layers=2, seed=7)
    model = _model_of(cache)
    g = torch.Generator().manual_seed(8)
    s1 = torch.rand(2, 2, 120, generator=g)
    cache.evict(1, s1.cuda(), budget=40, protected=6)           # request 1 now has a pinned mask
    model.evict(1, s1, budget=40, protected=6, tie_rule="lowest")
    _assert_same_state(cache, model)
    scores = [torch.rand(2, 2, cache.seq_used[r], generator=g) for r in range(3)]
    budgets, prots = [30, 20, 25], [5, 9, 0]
    perms = cache.evict_batch([0, 1, 2], [s.cuda() for s in scores], budgets, prots)
    for r in range(3):
        perm_o = model.evict(r, scores[r], budget=budgets[r], protected=prots[r], tie_rule="lowest")
        assert np.array_equal(perms[r].cpu().numpy(), perm_o), r
        assert np.array_equal(cache.pinned[r].cpu().numpy(), model.pinned[r]), r
    _assert_same_state(cache, model)


def test_per_request_evicts_after_one_batched_cal_attn_match_the_oracle():
    """The reference bench's step (benchmarks/bench_kernels.py:81-89): one cal_attn over every
    request, then evict of each request in a Python loop.  The evictions read their tables from
    the rows of the batch's device copy; the whole state still matches oracle evicts, also when
    a request grew after the batch's tables were uploaded (its row is stale and is not used)
    and when the loop runs a second time on the compacted cache."""
    lens = [300, 41, 517, 160]
    cache = _filled_cache(lens, hkv=2, d=32, layers=1, seed=31)
    model = _model_of(cache)
    g = torch.Generator().manual_seed(32)
    reqs = list(range(len(lens)))
    for rnd in range(2):
        q = torch.randn(len(reqs), 4, 32, generator=g).cuda()
        lse = torch.full((len(reqs), 4), 3.0, device="cuda")
        width = (max(len(cache.tables[r]) for r in reqs) + 4) * cache.block_size
        out = torch.zeros(len(reqs), 2, width, device="cuda")
        n_seen = torch.zeros(len(reqs), dtype=torch.int32, device="cuda")
        cache.cal_attn(reqs, q, lse, out, n_seen)
        if rnd == 1:   # request 2 grows after the batch's tables were uploaded (scores 0 there)
            k = torch.randn(1, 20, 2, 32, generator=g)
            cache.append(2, k.cuda(), k.cuda())
            model.append(2, _bits(k), _bits(k))
        scores = out.cpu()
        for r in reqs:
            budget = max(cache.seq_used[r] // 3, 1)
            perm = cache.evict(r, out[r], budget, protected=2)
            want = model.evict(r, scores[r, :, : model.seq_used[r]], budget, protected=2, tie_rule="lowest")
            assert np.array_equal(perm.cpu().numpy(), want), (rnd, r)
        _assert_same_state(cache, model)


def test_launches_follow_torch_current_stream():
    """The library launches on torch's current stream, including inside `torch.cuda.stream`."""
    from actkv import _hip
    dev = torch.device("cuda")
    assert _hip.stream(dev) == torch.cuda.current_stream().cuda_stream
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        assert _hip.stream(dev) == side.cuda_stream
        assert _hip.stream(torch.device("cuda", torch.cuda.current_device())) == side.cuda_stream
        # a scoring call queued on the side stream gives the same result as on the default one
        cache = _filled_cache([200, 150], hkv=2, d=128, layers=1, seed=11, dtype=torch.bfloat16)
        g = torch.Generator().manual_seed(12)
        q = torch.randn(2, 8, 128, generator=g).to(torch.bfloat16).cuda()
        lse = torch.full((2, 8), 6.0, device="cuda")
        width = max(len(cache.tables[r]) for r in (0, 1)) * cache.block_size
        a = torch.zeros(2, 2, width, device="cuda")
        na = torch.zeros(2, dtype=torch.int32, device="cuda")
        cache.cal_attn([0, 1], q, lse, a, na, layer=0)
    side.synchronize()
    b = torch.zeros_like(a)
    nb = torch.zeros_like(na)
    cache.cal_attn([0, 1], q, lse, b, nb, layer=0)
    assert torch.equal(a, b) and na.tolist() == nb.tolist() == [1, 1]


@pytest.mark.parametrize("n_q", [128, 8])
def test_scoring_interleaved_over_streams_counts_every_query_once(n_q):
    """Scoring calls interleaved over three streams (free to run concurrently, each with its own
    out and n_seen) count each call's queries once and leave the same running means, bit for
    bit, as the same calls on the default stream.  n_q = 128 runs the query-tile kernel
    (512 rows), 8 the K-slice kernel (32 rows)."""
    dev = torch.device("cuda")
    cache = _filled_cache([3000, 1700], hkv=8, d=128, layers=1, seed=21, dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(22)
    q = torch.randn(2, n_q, 32, 128, generator=g).to(torch.bfloat16).to(dev)
    lse = (6.0 + torch.rand(2, n_q, 32, generator=g)).to(dev)
    width = max(len(cache.tables[r]) for r in (0, 1)) * cache.block_size
    rounds = 4
    want = torch.zeros(2, 8, width, device=dev)
    n_want = torch.zeros(2, dtype=torch.int32, device=dev)
    for _ in range(rounds):
        cache.cal_attn([0, 1], q, lse, want, n_want)
    streams = [torch.cuda.Stream() for _ in range(3)]
    outs = [torch.zeros(2, 8, width, device=dev) for _ in streams]
    seen = [torch.zeros(2, dtype=torch.int32, device=dev) for _ in streams]
    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
    for _ in range(rounds):
        for st, o, n in zip(streams, outs, seen):
            with torch.cuda.stream(st):
                cache.cal_attn([0, 1], q, lse, o, n)
    for st in streams:
        st.synchronize()
    assert n_want.tolist() == [rounds * n_q] * 2
    for o, n in zip(outs, seen):
        assert n.tolist() == [rounds * n_q] * 2
        assert torch.equal(o, want)


def test_pinned_uploads_survive_ring_wraps_and_side_streams():
    """Host-to-device uploads through the pinned staging ring: enough of them to wrap the ring
    several times, every third queued on a side stream, and one larger than half the ring;
    every uploaded tensor holds its values."""
    from actkv import _hip
    dev = torch.device("cuda")
    ring = _hip._PinnedRing()
    side = torch.cuda.Stream()
    outs = []
    for i in range(1200):
        vals = list(range(i * 1000, i * 1000 + 700 + i % 5))
        if i % 3 == 0:
            with torch.cuda.stream(side):
                outs.append((vals, ring.upload_i32(vals, dev)))
        else:
            outs.append((vals, ring.upload_i32(vals, dev)))
    big = list(range(_hip._PinnedRing.SIZE // 2 + 10))
    outs.append((big, ring.upload_i32(big, dev)))
    torch.cuda.synchronize()
    for vals, t in outs:
        assert t.cpu().tolist() == vals


def test_pinned_uploads_that_fill_a_half_exactly():
    """Uploads whose sizes divide half the ring fill each half to its last entry: the next upload
    must change halves (waiting for the other half's copies) instead of running past the buffer
    or into the other half unchecked.  Three whole passes of the ring, then single uploads of
    exactly half the ring; every uploaded tensor holds its values."""
    from actkv import _hip
    dev = torch.device("cuda")
    ring = _hip._PinnedRing()
    half = _hip._PinnedRing.SIZE // 2
    n = 2048
    outs = []
    for i in range(3 * 2 * half // n + 5):
        vals = np.arange(i * n, (i + 1) * n, dtype=np.int32)
        outs.append((vals, ring.upload_i32(vals, dev)))
    for i in range(3):
        vals = np.full(half, i, dtype=np.int32)
        outs.append((vals, ring.upload_i32(vals, dev)))
    torch.cuda.synchronize()
    for vals, t in outs:
        assert np.array_equal(t.cpu().numpy(), vals)
