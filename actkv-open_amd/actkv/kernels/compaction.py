"""In-place KV cache compaction on a paged layout (ActKV Algorithm 4), on gfx950.

Drop-in for the reference module actkv/kernels/compaction.py.  A request of S tokens holds
Y = ceil(S / block_size) blocks; B survivors need X = ceil(B / block_size).  They end up in
the logical window [start, start + B) with start = (Y - X) * block_size: each hole of the
window (a non-kept position, ascending) receives the next survivor from outside the window
(ascending), so sources and destinations never overlap and every row move is independent of
the others.  The first Y - X logical blocks are then empty and go back to the allocator.

`plan_compaction` and `apply_copies` run HIP kernels of libactkv_hip.so (the planner is the
same kernel PagedKVCache.compact fuses with the moves, run with its copy phase off).  There
is no CPU path.  `apply_copies_ref` and `gather_compaction` are the reference's torch
formulations (compaction.py:72-74, :109-114), never called by the HIP path.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from .. import _hip

HAS_KERNELS = _hip.available()
HAS_TRITON = HAS_KERNELS


@dataclass
class CompactionPlan:
    src_slots: torch.Tensor   # physical slots to read
    dst_slots: torch.Tensor   # physical slots to write
    perm: torch.Tensor        # [B] new logical position -> old logical position
    drop_blocks: int          # leading logical blocks that become free (Y - X)


def upload_i32(values, device) -> torch.Tensor:
    """Host ints -> device int32 through reused pinned staging memory, without synchronising
    the stream."""
    return _hip.upload_i32(values, device)


def keep_words(seq_used: int, block_size: int) -> int:
    """uint32 words of packed keep bits for a request (whole blocks, LSB-first)."""
    return (math.ceil(seq_used / block_size) * block_size + 31) // 32


def plan_compaction(keep_mask: torch.Tensor, seq_used: int, block_table_row: torch.Tensor,
                    block_size: int) -> CompactionPlan:
    """Algorithm 4 steps 1-5 for one request. keep_mask: [>= seq_used] bool, True = retain.

    Reference: actkv/kernels/compaction.py:44-69.  Synchronises once (to size the outputs),
    as the reference does with int(keep.sum()) and torch.nonzero.
    """
    dev = _hip.require_gpu("plan_compaction", keep_mask, block_table_row)
    y = math.ceil(seq_used / block_size)
    if block_table_row.numel() < y:
        raise IndexError(f"block table has {block_table_row.numel()} entries, {y} needed")
    keep = keep_mask[:seq_used]
    if keep.dtype != torch.bool:
        keep = keep.bool()
    keep = keep.contiguous()
    bt = block_table_row.to(device=dev, dtype=torch.int32).contiguous().view(1, -1)
    seq = upload_i32([seq_used], dev)
    nw = keep_words(seq_used, block_size)
    bits = torch.empty(1, max(nw, 1), dtype=torch.int32, device=dev)
    st = _hip.stream(dev)
    lib = _hip.lib()
    _hip.check(lib.actkv_pack_keep(keep.data_ptr(), keep.numel(), 1, seq.data_ptr(), block_size,
                                   bits.data_ptr(), bits.shape[1], None, seq_used, st), "actkv_pack_keep")
    cap = max(seq_used, 1)
    perm = torch.empty(cap, dtype=torch.int64, device=dev)
    src = torch.empty(cap, dtype=torch.int64, device=dev)
    dst = torch.empty(cap, dtype=torch.int64, device=dev)
    counts = torch.empty(1, 4, dtype=torch.int32, device=dev)
    _hip.check(lib.actkv_compact(
        None, 0, 0, 0, 0, 2**31 - 1,
        bits.data_ptr(), bits.shape[1], 1, seq.data_ptr(),
        bt.data_ptr(), bt.shape[1], block_size,
        perm.data_ptr(), cap, None, 0, None, None, 0,
        None, 0, None, 0,
        src.data_ptr(), dst.data_ptr(), cap, counts.data_ptr(),
        0, seq_used, seq_used, st), "actkv_compact(plan)")
    b, m, drop, _x = counts[0].tolist()
    return CompactionPlan(src[:m], dst[:m], perm[:b], drop)


def apply_copies_ref(kv_flat: torch.Tensor, src: torch.Tensor, dst: torch.Tensor) -> None:
    """kv_flat [N, slots, H*D]: row dst[i] of every plane receives row src[i], in torch.
    src and dst are disjoint, so reading every source before writing is the same as moving
    the rows one by one.

    Reference formulation: actkv/kernels/compaction.py:72-74.
    """
    kv_flat.index_copy_(1, dst.to(kv_flat.device), kv_flat.index_select(1, src.to(kv_flat.device)))


def apply_copies(kv_flat: torch.Tensor, src: torch.Tensor, dst: torch.Tensor) -> None:
    """kv_flat[p, dst[i], :] = kv_flat[p, src[i], :] for every plane p (HIP, in place).

    Reference: actkv/kernels/compaction.py:96-106.
    """
    if src.numel() == 0:
        return
    dev = _hip.require_gpu("apply_copies", kv_flat, src, dst)
    planes, slots, row = kv_flat.shape
    assert kv_flat.stride(2) == 1
    if src.numel() != dst.numel():
        raise ValueError(f"{src.numel()} sources but {dst.numel()} destinations")
    s = src.to(device=dev, dtype=torch.int64).contiguous()
    d = dst.to(device=dev, dtype=torch.int64).contiguous()
    es = kv_flat.element_size()
    _hip.check(_hip.lib().actkv_copy_slots(kv_flat.data_ptr(), planes, kv_flat.stride(0) * es,
                                           kv_flat.stride(1) * es, row * es, slots, s.data_ptr(),
                                           d.data_ptr(), s.numel(), _hip.stream(dev)),
               "actkv_copy_slots")


def gather_compaction(kv_flat: torch.Tensor, keep_slots: torch.Tensor) -> torch.Tensor:
    """Gather-based baseline (paged R-KV style): the survivors' rows of every plane copied into
    a fresh contiguous buffer [N, len(keep_slots), H*D].

    Reference formulation: actkv/kernels/compaction.py:109-114 (benchmark comparison only).
    """
    return kv_flat.index_select(1, keep_slots.to(kv_flat.device))
