"""Host-side logic of the drop-in modules that needs no GPU: allocator bookkeeping, the block
table mirror, argument validation with the reference's exceptions, and the rule that the HIP
entry points refuse CPU tensors (there is no CPU fallback)."""
import math

import numpy as np
import pytest
import torch

from actkv.kernels import compaction, lse_attn
from actkv.paged import OutOfBlocks, PagedKVCache, _Table, keep_mask_from_scores


def test_table_counts_mutations_and_keeps_its_mirror():
    t = _Table([5, 3, 9])
    assert t.as_array().tolist() == [5, 3, 9] and t.as_array().dtype == np.int32
    v = t.version
    for op in (lambda x: x.append(7), lambda x: x.extend([1, 2]), lambda x: x.__setitem__(0, 11),
               lambda x: x.pop(), lambda x: x.insert(1, 4), lambda x: x.remove(4), lambda x: x.reverse(),
               lambda x: x.sort(), lambda x: x.__delitem__(0), lambda x: x.__iadd__([8])):
        op(t)
        assert t.version > v
        v = t.version
        assert t.as_array().tolist() == list(t)
    t.extend_ids([40, 41])
    assert t.as_array().tolist() == list(t)
    tail = t.tail(2)
    assert isinstance(tail, _Table) and list(tail) == list(t)[2:] and tail.as_array().tolist() == list(t)[2:]
    assert isinstance(t[1:], list)


def _grow(cache, req, n):
    """The host side of append (paged.py:76-79, 84): blocks for n more tokens, then the length."""
    start = cache.seq_used.get(req, 0)
    cache._ensure(req, start + n)
    cache.seq_used[req] = start + n


def test_allocator_matches_the_reference_stack_order():
    """free is a stack popped from the end; release pushes reversed (paged.py:56, :73-74, :88)."""
    cache = PagedKVCache(10, 4, 1, 2, n_layers=1, dtype=torch.float32, device="cpu")
    _grow(cache, 0, 9)
    assert cache.tables[0] == [0, 1, 2] and cache.used_blocks == 3
    _grow(cache, 1, 1)
    assert cache.tables[1] == [3]
    _grow(cache, 0, 4)                                                # 13 tokens -> 4 blocks
    assert cache.tables[0] == [0, 1, 2, 4] and cache.seq_used[0] == 13
    assert cache.tables[0].as_array().tolist() == [0, 1, 2, 4]
    cache.release(0)
    assert cache.free[-4:] == [4, 2, 1, 0] and 0 not in cache.tables
    _grow(cache, 2, 5)
    assert cache.tables[2] == [0, 1]
    with pytest.raises(OutOfBlocks):
        _grow(cache, 3, 40)


def test_data_movement_needs_a_gpu_cache():
    """append, slot_map and gather run HIP kernels; a CPU-resident cache raises instead of
    taking a torch path (there is one implementation of each)."""
    cache = PagedKVCache(8, 4, 2, 3, n_layers=2, dtype=torch.float32, device="cpu")
    k = torch.zeros(2, 10, 2, 3)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        cache.append(0, k, k)
    assert cache.seq_used.get(0, 0) == 0 and cache.used_blocks == 0
    _grow(cache, 0, 10)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        cache.slot_map(0)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        cache.gather(0, layer=1)


def test_host_table_layout():
    cache = PagedKVCache(12, 4, 1, 2, device="cpu", dtype=torch.float32)
    _grow(cache, 0, 9)
    _grow(cache, 1, 2)
    host, mb = cache._host_tables([1, 0])
    assert mb == 3 and host[:2].tolist() == [2, 9]
    assert host[2:].reshape(2, 3).tolist() == [[3, 0, 0], [0, 1, 2]]
    assert cache.block_table([0, 1]).tolist() == [[0, 1, 2], [3, 0, 0]]
    assert cache.seq_tensor([0, 1]).tolist() == [9, 2]


def test_action_scores_rejects_a_buffer_narrower_than_the_cache():
    """The reference raises ValueError("...wide...") before launching (lse_attn.py:139-142)."""
    kv = torch.zeros(2, 4, 16, 2, 16)
    bt = torch.zeros(1, 3, dtype=torch.int32)
    out = torch.zeros(1, 2, 16)
    with pytest.raises(ValueError, match="wide"):
        lse_attn.action_scores(torch.zeros(1, 4, 16), kv, bt, torch.tensor([40], dtype=torch.int32),
                               torch.zeros(1, 4), out, torch.zeros(1, dtype=torch.int32))


def test_kernel_entry_points_refuse_cpu_tensors():
    kv = torch.zeros(2, 4, 16, 2, 16)
    bt = torch.zeros(1, 3, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        lse_attn.action_scores(torch.zeros(1, 4, 16), kv, bt, torch.tensor([40], dtype=torch.int32),
                               torch.zeros(1, 4), torch.zeros(1, 2, 48), torch.zeros(1, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        compaction.apply_copies(torch.zeros(2, 10, 4), torch.tensor([1]), torch.tensor([2]))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        compaction.plan_compaction(torch.ones(5, dtype=torch.bool), 5, torch.tensor([0]), 16)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        keep_mask_from_scores(torch.rand(2, 10), 10, 3)
    cache = PagedKVCache(4, 16, 1, 4, device="cpu", dtype=torch.float32)
    _grow(cache, 0, 20)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        cache.compact(0, torch.ones(20, dtype=torch.bool))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        cache.evict(0, torch.rand(20), budget=3)


def test_keep_mask_rejects_an_unknown_head_reduce():
    with pytest.raises(ValueError):
        keep_mask_from_scores(torch.rand(2, 10), 10, 3, head_reduce="median")


def test_apply_copies_with_no_pairs_is_a_no_op_anywhere():
    compaction.apply_copies(torch.zeros(2, 10, 4), torch.tensor([], dtype=torch.long), torch.tensor([], dtype=torch.long))


def test_evict_within_budget_needs_no_kernel():
    """A request already within budget returns arange(n) untouched (paged.py:153-154)."""
    cache = PagedKVCache(4, 16, 1, 4, device="cpu", dtype=torch.float32)
    _grow(cache, 0, 20)
    table = list(cache.tables[0])
    assert cache.evict(0, torch.rand(20), budget=20).tolist() == list(range(20))
    assert cache.tables[0] == table and cache.seq_used[0] == 20
    assert cache.pinned[0].tolist() == [False] * 20


def test_evict_batch_takes_each_request_once():
    cache = PagedKVCache(8, 16, 1, 4, device="cpu", dtype=torch.float32)
    _grow(cache, 0, 40)
    with pytest.raises(ValueError, match="once"):
        cache.evict_batch([0, 0], [torch.rand(40), torch.rand(40)], budget=10)
    assert cache.seq_used[0] == 40 and len(cache.tables[0]) == 3


def test_evict_refuses_pins_longer_than_the_request():
    """After a compact() the stored pins are longer than the request; the reference's pad
    with a negative length raises (paged.py:151), and so does evict here."""
    cache = PagedKVCache(8, 16, 1, 4, device="cpu", dtype=torch.float32)
    _grow(cache, 0, 20)
    cache.pinned[0] = torch.zeros(25, dtype=torch.bool)
    with pytest.raises(RuntimeError, match="pinned"):
        cache.evict(0, torch.rand(20), budget=30)


def test_head_reduce_is_checked_after_the_within_budget_return():
    """paged.py:149-155: a request within budget returns arange(n) before keep_mask_from_scores
    sees head_reduce; over budget, an unknown reduction raises ValueError."""
    cache = PagedKVCache(8, 16, 1, 4, device="cpu", dtype=torch.float32)
    _grow(cache, 0, 20)
    assert cache.evict(0, torch.rand(20), budget=20, head_reduce="median").tolist() == list(range(20))
    with pytest.raises(ValueError, match="median"):
        cache.evict(0, torch.rand(20), budget=5, head_reduce="median")


def test_lrfu_buffers_cover_whole_blocks():
    """A max_tokens that is not a multiple of the block size still leaves cal_attn an output
    as wide as the block table spans (lse_attn.py:139-142)."""
    from actkv.kernels.lrfu import PagedLRFU
    cache = PagedKVCache(80, 16, 2, 4, n_layers=3, device="cpu", dtype=torch.float32)
    lr = PagedLRFU(cache, [0, 1], 500)
    assert lr.scores.shape == (3, 2, 2, 512) and lr.ks.shape == (3, 2, 512) and lr.pins.shape == (2, 512)
    assert lr.max_tokens == 500


def _plan_outputs(keep, seq, table, bs):
    """The report and plan actkv_compact writes for one request, from the oracle's planner."""
    from oracle import reference as ref
    src, dst, perm, drop = ref.plan_compaction(keep, seq, table, bs)
    b = int(np.asarray(keep[:seq]).sum())
    return np.array([b, src.size, drop, -(-b // bs)], dtype=np.int32), src, dst


def test_debug_compaction_check_accepts_a_correct_plan_and_catches_a_wrong_one():
    from actkv.paged import _check_compaction
    rng = np.random.default_rng(0)
    bs, seqs = 16, [200, 77]
    keeps = [rng.random(s) < 0.3 for s in seqs]
    tables = [list(range(13)), list(range(13, 18))]
    words = np.zeros((2, 8), dtype=np.uint32)
    counts = np.zeros((2, 4), dtype=np.int32)
    src = np.full((2, 200), -1, dtype=np.int64)
    dst = np.full((2, 200), -1, dtype=np.int64)
    for i, (k, s) in enumerate(zip(keeps, seqs)):
        padded = np.zeros(256, dtype=bool)
        padded[:s] = k
        words[i] = np.packbits(padded, bitorder="little").view(np.uint32)[:8]
        counts[i], ps, pd = _plan_outputs(k, s, tables[i], bs)
        src[i, : ps.size], dst[i, : pd.size] = ps, pd
    kept = [int(k.sum()) for k in keeps]
    args = (torch.from_numpy(words.view(np.int32)), torch.from_numpy(counts), torch.from_numpy(src),
            torch.from_numpy(dst))
    _check_compaction([0, 1], seqs, kept, bs, *args)
    with pytest.raises(RuntimeError, match="host expects"):
        _check_compaction([0, 1], seqs, [kept[0] + 1, kept[1]], bs, *args)
    bad = counts.copy()
    bad[1] = -1
    with pytest.raises(RuntimeError, match="sized"):
        _check_compaction([0, 1], seqs, kept, bs, args[0], torch.from_numpy(bad), args[2], args[3])
    m = counts[0, 1]
    if m >= 2:
        clash = dst.copy()
        clash[0, 1] = src[0, 0]
        with pytest.raises(RuntimeError, match="disjoint"):
            _check_compaction([0, 1], seqs, kept, bs, args[0], args[1], args[2], torch.from_numpy(clash))


@pytest.mark.parametrize("shape,perm,dtype,seq", [
    ((300,), None, torch.float32, 257),                      # [W]
    ((8, 300), None, torch.float32, 300),                    # [Hkv, W]
    ((3, 8, 300), None, torch.bfloat16, 290),                # [L, Hkv, W]
    ((2, 3, 8, 300), None, torch.float16, 111),              # [L1, L2, Hkv, W]: the leading dims collapse
    ((3, 8, 300), (1, 0, 2), torch.float32, 200),            # heads outermost in memory: still a stride pair
    ((8, 300, 3), (2, 0, 1), torch.float32, 300),            # [L, Hkv, W] view of a W-major buffer: copied
    ((2, 3, 8, 300), (1, 0, 2, 3), torch.float32, 64),       # leading dims that do not collapse: copied
    ((3, 8, 300), None, torch.float64, 150),                 # not a kernel dtype: converted
])
def test_scores_layout_addresses_the_same_scores(shape, perm, dtype, seq):
    """The eviction reads scores in place through (L, H, layer stride, head stride) with a unit
    last stride: the geometry it derives must address exactly scores[..., h, t] for t < seq,
    whether the tensor is used as it is or copied first."""
    from actkv.paged import _scores_layout
    g = torch.Generator().manual_seed(len(shape) * 1000 + seq)
    base = torch.rand(*shape, generator=g).to(dtype)
    scores = base.permute(*perm) if perm else base
    t, L, H, s_sl, s_sh = _scores_layout(scores, seq)
    assert t.dtype in (torch.float32, torch.float16, torch.bfloat16) and t.stride(-1) == 1
    want = scores[..., :seq].reshape(L, H, seq).to(t.dtype)
    got = torch.as_strided(t, (L, H, seq), (s_sl, s_sh, 1), t.storage_offset())
    assert torch.equal(got, want)
    with pytest.raises(ValueError):
        _scores_layout(scores, scores.shape[-1] + 1)
