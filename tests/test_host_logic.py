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


def test_allocator_matches_the_reference_stack_order():
    """free is a stack popped from the end; release pushes reversed (paged.py:56, :73-74, :88)."""
    cache = PagedKVCache(10, 4, 1, 2, n_layers=1, dtype=torch.float32, device="cpu")
    cache.append(0, torch.zeros(1, 9, 1, 2), torch.zeros(1, 9, 1, 2))
    assert cache.tables[0] == [0, 1, 2] and cache.used_blocks == 3
    cache.append(1, torch.zeros(1, 1, 1, 2), torch.zeros(1, 1, 1, 2))
    assert cache.tables[1] == [3]
    cache.append(0, torch.ones(1, 4, 1, 2), torch.ones(1, 4, 1, 2))   # 13 tokens -> 4 blocks
    assert cache.tables[0] == [0, 1, 2, 4] and cache.seq_used[0] == 13
    assert cache.tables[0].as_array().tolist() == [0, 1, 2, 4]
    cache.release(0)
    assert cache.free[-4:] == [4, 2, 1, 0] and 0 not in cache.tables
    cache.append(2, torch.zeros(1, 5, 1, 2), torch.zeros(1, 5, 1, 2))
    assert cache.tables[2] == [0, 1]
    with pytest.raises(OutOfBlocks):
        cache.append(3, torch.zeros(1, 40, 1, 2), torch.zeros(1, 40, 1, 2))


def test_gather_and_slot_map_follow_the_block_table():
    cache = PagedKVCache(8, 4, 2, 3, n_layers=2, dtype=torch.float32, device="cpu")
    cache.free = [7, 2, 5, 0, 1, 3, 6, 4]
    k = torch.arange(2 * 10 * 2 * 3, dtype=torch.float32).view(2, 10, 2, 3)
    cache.append(0, k, -k)
    assert cache.tables[0] == [4, 6, 3]
    slots = cache.slot_map(0)
    assert slots.tolist() == [16, 17, 18, 19, 24, 25, 26, 27, 12, 13]
    kk, vv = cache.gather(0, layer=1)
    assert torch.equal(kk, k[1]) and torch.equal(vv, -k[1])


def test_host_table_layout():
    cache = PagedKVCache(12, 4, 1, 2, device="cpu", dtype=torch.float32)
    cache.append(0, torch.zeros(1, 9, 1, 2), torch.zeros(1, 9, 1, 2))
    cache.append(1, torch.zeros(1, 2, 1, 2), torch.zeros(1, 2, 1, 2))
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
    cache.append(0, torch.zeros(1, 20, 1, 4), torch.zeros(1, 20, 1, 4))
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
    cache.append(0, torch.zeros(1, 20, 1, 4), torch.zeros(1, 20, 1, 4))
    table = list(cache.tables[0])
    assert cache.evict(0, torch.rand(20), budget=20).tolist() == list(range(20))
    assert cache.tables[0] == table and cache.seq_used[0] == 20
    assert cache.pinned[0].tolist() == [False] * 20
