"""A vLLM-style paged KV cache whose eviction primitives run on gfx950 HIP kernels.

    kv[layer] : [2, num_blocks, block_size, n_kv_heads, head_dim]

Drop-in for the reference module actkv/paged.py (same class, attributes, methods and
errors).  The allocator state (`free`, `tables`, `seq_used`, `pinned`) stays in host Python
lists and dicts exactly as in the reference, so callers may read and assign it; the device
work of `cal_attn`, `keep_mask_from_scores`, `compact` and `evict` runs in libactkv_hip.so:

  cal_attn   -> actkv_action_scores  (Algorithm 3, N action tokens and L layers per launch)
  evict      -> actkv_keep_mask      (head/layer reduction, radix top-k, keep bits)
             -> actkv_compact        (plan + conflict-free moves + reclaim, one launch)

`evict` does not synchronise the device: the kept count B is known on the host (protected
count + budget), so the host lists are updated from host values while the kernels run.
`compact` with a caller-supplied mask synchronises once to learn B, as the reference does.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from . import _hip
from .kernels.compaction import keep_words, upload_i32
from .kernels.lse_attn import action_scores, paged_decode_attention


class OutOfBlocks(RuntimeError):
    pass


class _Table(list):
    """A request's block table: a plain list of physical block ids (callers may read, copy and
    mutate it like the reference's) that counts its own mutations and keeps an int32 mirror,
    so the device copy of an unchanged table is reused instead of re-converted and re-sent."""

    __slots__ = ("version", "_np", "_np_version")

    def __init__(self, it=(), mirror=None):
        super().__init__(it)
        self.version = 0
        self._np, self._np_version = mirror, 0

    def as_array(self) -> np.ndarray:
        if self._np is None or self._np_version != self.version or self._np.size != len(self):
            self._np = np.array(self, dtype=np.int32)
            self._np_version = self.version
        return self._np

    def extend_ids(self, ids) -> None:
        """Append newly allocated blocks and grow the mirror instead of rebuilding it."""
        fresh = self._np is not None and self._np_version == self.version and self._np.size == len(self)
        super().extend(ids)
        self.version += 1
        if fresh:
            self._np = np.concatenate([self._np, np.asarray(ids, dtype=np.int32)])
            self._np_version = self.version

    def tail(self, drop: int) -> "_Table":
        """A new table holding self[drop:] (the survivors of a compaction), mirror sliced."""
        arr = self.as_array()
        return _Table(self[drop:], arr[drop:])


def _mutator(name):
    base = getattr(list, name)

    def method(self, *args, **kw):
        self.version += 1
        return base(self, *args, **kw)

    method.__name__ = name
    return method


for _name in ("__setitem__", "__delitem__", "__iadd__", "__imul__", "append", "extend", "insert", "pop",
              "remove", "clear", "sort", "reverse"):
    setattr(_Table, _name, _mutator(_name))


def _as_i32(table) -> np.ndarray:
    return table.as_array() if isinstance(table, _Table) else np.array(table, dtype=np.int32)


_REDUCE = {"mean": _hip.REDUCE_MEAN, "max": _hip.REDUCE_MAX}


_SCORE_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def _scores_layout(scores: torch.Tensor, seq_used: int):
    """[..., H, W] / [H, W] / [W] -> (tensor, L, H, s_sl, s_sh) with a unit last stride.

    The kernels read columns [0, seq_used) of each row through the strides, so a tensor of a
    kernel dtype with a unit last stride, whose leading dims collapse into one layer stride, is
    used as it is: no view is built (each costs host time on every eviction).  Other dtypes and
    layouts are copied first, their seq_used columns only."""
    shape = scores.shape
    nd = len(shape)
    if shape[-1] < seq_used:
        raise ValueError(f"scores cover {shape[-1]} tokens, seq_used is {seq_used}")
    st = scores.stride()
    if scores.dtype in _SCORE_DTYPES and st[-1] == 1:
        if nd == 1:
            return scores, 1, 1, 0, 0
        if nd == 2:
            return scores, 1, shape[0], 0, st[0]
        if nd == 3:
            return scores, shape[0], shape[1], st[0], st[1]
        if all(st[i] == st[i + 1] * shape[i + 1] for i in range(nd - 3)):
            return scores, math.prod(shape[:-2]), shape[-2], st[nd - 3], st[-2]
    s = scores[..., :seq_used]
    if s.dtype not in _SCORE_DTYPES:
        s = s.float()
    if s.stride(-1) != 1:
        s = s.contiguous()
    if s.dim() == 1:
        return s, 1, 1, 0, 0
    if s.dim() == 2:
        return s, 1, s.shape[0], 0, s.stride(0)
    h = s.shape[-2]
    try:
        s3 = s.view(-1, h, seq_used)
    except RuntimeError:
        s3 = s.reshape(-1, h, seq_used).contiguous()
    return s3, s3.shape[0], h, s3.stride(0), s3.stride(1)


def _keep_mask_launch(s, L, H, s_sl, s_sr, s_sh, R, seq_dev, budget_dev, prot_count_dev,
                      prot_mask, pm_sr, head_reduce, block_size, max_seq, device, want_keep=True):
    """Run actkv_keep_mask; returns (keep [R, max_seq] bool or None, bits [R, words] int32)."""
    keep = torch.empty(R, max(max_seq, 1), dtype=torch.bool, device=device) if want_keep else None
    nw = keep_words(max_seq, block_size)
    bits = torch.empty(R, max(nw, 1), dtype=torch.int32, device=device)
    ws = _hip.workspace(device, _hip.WS_KEEP_MASK, R, max_seq)
    rc = _hip.glue().keep_mask(
        s.data_ptr(), _hip.dtype_code(s.dtype), s_sl, s_sr, s_sh, L, H, R,
        seq_dev.data_ptr(), budget_dev.data_ptr(), _hip.ptr(prot_count_dev), _hip.ptr(prot_mask), pm_sr,
        _REDUCE[head_reduce], _hip.ptr(keep), 0 if keep is None else keep.shape[1], bits.data_ptr(),
        bits.shape[1], block_size, max_seq, ws.data_ptr(), ws.numel(), _hip.stream(device))
    _hip.check(rc, "actkv_keep_mask")
    return keep, bits


def _keep_mask_bits(scores, seq_used: int, budget: int, protected, head_reduce: str, block_size: int):
    if head_reduce not in _REDUCE:
        raise ValueError(head_reduce)
    dev = _hip.require_gpu("keep_mask_from_scores", scores,
                           protected if isinstance(protected, torch.Tensor) else None)
    s, L, H, s_sl, s_sh = _scores_layout(scores, seq_used)
    prot_mask = None
    if isinstance(protected, torch.Tensor):
        prot_mask = protected.to(device=dev, dtype=torch.bool)
        if prot_mask.numel() < seq_used:
            raise ValueError(f"protected mask has {prot_mask.numel()} entries, seq_used is {seq_used}")
        prot_mask = prot_mask.reshape(-1).contiguous()
        params = upload_i32([seq_used, budget], dev)
        prot_count = None
    else:
        params = upload_i32([seq_used, budget, int(protected)], dev)
        prot_count = params[2:3]
    return _keep_mask_launch(s, L, H, s_sl, 0, s_sh, 1, params[0:1], params[1:2], prot_count,
                             prot_mask, 0, head_reduce, block_size, seq_used, dev)


def keep_mask_from_scores(scores: torch.Tensor, seq_used: int, budget: int,
                          protected: int | torch.Tensor = 0, head_reduce: str = "mean") -> torch.Tensor:
    """Per-token scores -> keep mask [seq_used]: the protected tokens plus the top-`budget` others.

    scores: [S], [Hkv, S] or [n_layers, Hkv, S].  KV heads are reduced with `head_reduce`, then
    layers are averaged (float32, in torch's CPU summation order, so the per-token score is
    bit-identical to the reference's).  protected: a count of leading tokens, or a bool mask
    [seq_used] of tokens that are always kept.  Equal scores at the top-k boundary keep the
    lower index.

    Reference: actkv/paged.py:23-46.
    """
    keep, _ = _keep_mask_bits(scores, seq_used, budget, protected, head_reduce, 16)
    return keep[0, :seq_used]


def _check_compaction(reqs, seqs, kept, block_size, bits, counts, src, dst) -> None:
    """Debug-mode check of one actkv_compact launch (synchronises): the kernel's report
    {B, M, drop, X} per request must equal the host's counts (reference compaction.py:48-52,
    :61) and the plan's source and destination slots must be distinct and disjoint
    (compaction.py:3-13), which is what makes the in-place moves order-free."""
    rep = counts.cpu().numpy()
    words = bits.cpu().numpy().astype(np.uint32)
    src_h, dst_h = src.cpu().numpy(), dst.cpu().numpy()
    for i, r in enumerate(reqs):
        b, m, drop, x = (int(v) for v in rep[i])
        if b == -1:
            raise RuntimeError(f"actkv_compact: request {r} keeps more tokens than the launch was sized for")
        if b == -2:
            raise RuntimeError(f"actkv_compact: request {r} holds more tokens than the launch's max_seq")
        s = seqs[i]
        y = -(-s // block_size)
        mask = np.unpackbits(words[i].view(np.uint8), bitorder="little")[: y * block_size].astype(bool)
        if mask[s:].any():
            raise RuntimeError(f"actkv_compact: request {r} has keep bits past its {s} tokens")
        want_x = -(-kept[i] // block_size)
        start = (y - want_x) * block_size
        want_m = int(mask[:start].sum()) + int(mask[start + kept[i]:].sum())
        if (b, m, drop, x) != (kept[i], want_m, y - want_x, want_x) or int(mask.sum()) != kept[i]:
            raise RuntimeError(f"actkv_compact: request {r}: device reports B={b} M={m} drop={drop} X={x}, "
                               f"host expects B={kept[i]} M={want_m} drop={y - want_x} X={want_x} "
                               f"(keep bits hold {int(mask.sum())})")
        ps, pd = src_h[i, :m], dst_h[i, :m]
        if (ps < 0).any() or (pd < 0).any():
            raise RuntimeError(f"actkv_compact: request {r}: a move outside the block pool")
        if np.unique(ps).size != m or np.unique(pd).size != m or np.intersect1d(ps, pd).size:
            raise RuntimeError(f"actkv_compact: request {r}: source and destination slots are not "
                               "distinct and disjoint")


class PagedKVCache:
    def __init__(self, num_blocks: int, block_size: int, n_kv_heads: int, head_dim: int,
                 n_layers: int = 1, dtype=torch.float16, device="cpu"):
        self.block_size, self.n_kv_heads, self.head_dim = block_size, n_kv_heads, head_dim
        self.n_layers, self.num_blocks = n_layers, num_blocks
        self.kv = torch.zeros(n_layers, 2, num_blocks, block_size, n_kv_heads, head_dim,
                              dtype=dtype, device=device)
        self.free: list[int] = list(range(num_blocks - 1, -1, -1))
        self.tables: dict[int, list[int]] = {}
        self.seq_used: dict[int, int] = {}
        self.pinned: dict[int, torch.Tensor] = {}   # per request: which logical positions evict() protects
        self.device = device
        self._pin_count: dict[int, tuple] = {}      # req -> (tensor, version, count): avoids a sync
        self._dev_cache: dict = {}                  # device copies of unchanged block tables
        self._dev_rows: dict = {}                   # req -> (batch entry key, row) of _dev_cache
        self._const_cache: dict = {}                # device copies of budget / protected-count lists
        self._kv_dev = self.kv.device               # keys the two device caches by stream

    # ---------------------------------------------------------------- allocation
    @property
    def used_blocks(self) -> int:
        return self.num_blocks - len(self.free)

    def _ensure(self, req: int, n_tokens: int) -> None:
        table = self.tables.setdefault(req, _Table())
        self.seq_used.setdefault(req, 0)
        need = math.ceil(n_tokens / self.block_size) - len(table)
        if need > len(self.free):
            raise OutOfBlocks(f"need {need} blocks, {len(self.free)} free")
        if need > 0:
            ids = [self.free.pop() for _ in range(need)]
            if isinstance(table, _Table):
                table.extend_ids(ids)
            else:
                table.extend(ids)

    def append(self, req: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """k, v: [n_layers, n, Hkv, D] new tokens for request `req`.

        On a GPU cache one actkv_append launch writes every layer's K and V rows (converted to
        the cache dtype); the blocks come from the host free stack first, as in the reference.
        Reference: actkv/paged.py:76-84."""
        _hip.require_gpu("PagedKVCache.append", self.kv)
        n = k.shape[1]
        start = self.seq_used.get(req, 0)
        self._ensure(req, start + n)
        self._append_device([req], [start], [n], k, v)
        self.seq_used[req] = start + n

    def append_batch(self, reqs, k: torch.Tensor, v: torch.Tensor, counts=None) -> None:
        """Append to several requests in one launch: k, v [n_layers, sum(counts), Hkv, D] hold
        the requests' new tokens back to back (counts defaults to one token each, a decode
        step).  Blocks are allocated request by request in the order given, so the free stack
        ends exactly as after the same append() calls in a loop.  GPU caches only."""
        reqs = list(reqs)
        counts = [1] * len(reqs) if counts is None else [int(c) for c in counts]
        if len(counts) != len(reqs) or len(set(reqs)) != len(reqs):
            raise ValueError("append_batch: one count per request, each request once")
        if sum(counts) != k.shape[1] or v.shape[1] != k.shape[1]:
            raise ValueError(f"append_batch: k/v hold {k.shape[1]} tokens, counts sum to {sum(counts)}")
        _hip.require_gpu("PagedKVCache.append_batch", self.kv)
        starts = []
        for r, c in zip(reqs, counts):
            start = self.seq_used.get(r, 0)
            self._ensure(r, start + c)
            starts.append(start)
        self._append_device(reqs, starts, counts, k, v)
        for r, s0, c in zip(reqs, starts, counts):
            self.seq_used[r] = s0 + c

    def _append_src(self, x: torch.Tensor, total: int, n_layers: int | None = None) -> torch.Tensor:
        """A source operand as [L, total, Hkv, D] on the cache's device with a unit last stride
        (broadcasting like the reference's indexed assignment); dtypes the kernel does not read
        are converted to the cache dtype first, which is the reference's own conversion."""
        x = x.to(device=self.kv.device)
        if x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            x = x.to(self.kv.dtype)
        n_l = self.n_layers if n_layers is None else n_layers
        x = torch.broadcast_to(x, (n_l, total, self.n_kv_heads, self.head_dim))
        return x if x.stride(-1) == 1 else x.contiguous()

    def _append_device(self, reqs, starts, counts, k, v) -> None:
        total = sum(counts)
        if total == 0:
            return
        self._append_launch(self._append_plan(reqs, starts, counts), k, v)

    def _append_plan(self, reqs, starts, counts):
        """The device side of an append whose blocks are allocated: one upload of the source
        offsets (int64, as lo/hi int32 pairs), start positions, counts and block tables.
        Reused by every launch of the same step (a model writes one layer at a time)."""
        r_n = len(reqs)
        tabs = [_as_i32(self.tables[r]) for r in reqs]
        mb = max(max(t.size for t in tabs), 1)
        host = np.zeros(4 * r_n + r_n * mb, dtype=np.int32)
        off = np.concatenate([[0], np.cumsum(counts[:-1])]).astype(np.int64)
        host[: 2 * r_n] = off.view(np.int32)
        host[2 * r_n: 3 * r_n] = starts
        host[3 * r_n: 4 * r_n] = counts
        grid = host[4 * r_n:].reshape(r_n, mb)
        for i, t in enumerate(tabs):
            grid[i, : t.size] = t
        return self._upload(host), r_n, mb, int(sum(counts))

    def _append_launch(self, plan, k, v, layer=None) -> None:
        """k, v [L, total, Hkv, D] (or [1, total, Hkv, D] for one `layer`) -> the cache."""
        dev, r_n, mb, total = plan
        if total == 0:
            return
        if k.dtype != v.dtype:
            # one source dtype per launch: convert both as the reference does, straight to the
            # cache dtype (through the other source dtype could round twice)
            k, v = k.to(self.kv.dtype), v.to(self.kv.dtype)
        n_l = self.n_layers if layer is None else 1
        k = self._append_src(k, total, n_l)
        v = self._append_src(v, total, n_l)
        kv = self.kv if layer is None else self.kv[layer:layer + 1]
        if kv.stride(-1) != 1:
            raise RuntimeError("PagedKVCache.kv must have a unit last stride")
        rc = _hip.lib().actkv_append(
            kv.data_ptr(), _hip.dtype_code(kv.dtype), kv.stride(0), kv.stride(1), kv.stride(2),
            kv.stride(3), kv.stride(4), self.num_blocks,
            k.data_ptr(), v.data_ptr(), _hip.dtype_code(k.dtype),
            k.stride(0), k.stride(1), k.stride(2), v.stride(0), v.stride(1), v.stride(2),
            n_l, self.n_kv_heads, self.head_dim, r_n,
            dev[2 * r_n:].data_ptr(), dev[3 * r_n:].data_ptr(), dev.data_ptr(), total,
            dev[4 * r_n:].data_ptr(), mb, mb, self.block_size, None, _hip.stream(kv.device))
        _hip.check(rc, "actkv_append")

    def release(self, req: int) -> None:
        self.free.extend(reversed(self.tables.pop(req, [])))
        self.seq_used.pop(req, None)
        self.pinned.pop(req, None)
        self._pin_count.pop(req, None)

    # ---------------------------------------------------------------- views
    def slot_map(self, req: int, n: int | None = None) -> torch.Tensor:
        """Physical slot of each of the first n logical positions (int64 [n]); on a GPU cache
        computed by actkv_slot_map from the request's device block table.
        Reference: actkv/paged.py:93-97."""
        _hip.require_gpu("PagedKVCache.slot_map", self.kv)
        n = self.seq_used[req] if n is None else n
        table = self.tables[req]
        if n < 0 or n > len(table) * self.block_size:
            raise IndexError(f"slot_map: {n} positions, the table covers {len(table) * self.block_size}")
        out = torch.empty(n, dtype=torch.long, device=self.kv.device)
        if n == 0:
            return out
        _, bt = self._device_tables([req])
        rc = _hip.lib().actkv_slot_map(bt.data_ptr(), bt.shape[1], 0, n, self.block_size, out.data_ptr(),
                                       _hip.stream(self.kv.device))
        _hip.check(rc, "actkv_slot_map")
        return out

    def _host_tables(self, reqs, ys=None):
        """[len(reqs) + R*MB] int32 host array: seq_used values, then the block tables (first
        ys[i] entries of each, zero padded to MB columns)."""
        tabs = [_as_i32(self.tables[r]) for r in reqs]
        if ys is None:
            ys = [t.size for t in tabs]
        mb = max(max(ys), 1)
        r_n = len(reqs)
        host = np.zeros(r_n + r_n * mb, dtype=np.int32)
        host[:r_n] = [self.seq_used[r] for r in reqs]
        grid = host[r_n:].reshape(r_n, mb)
        for i, t in enumerate(tabs):
            grid[i, : ys[i]] = t[: ys[i]]
        return host, mb

    def _upload(self, host: np.ndarray) -> torch.Tensor:
        if torch.device(self.device).type != "cuda":
            return torch.from_numpy(host.copy()).to(self.device)
        return _hip.upload_i32(host, torch.device(self.device))

    def _device_tables(self, reqs, ys=None, shared_rows=False):
        """(seq_used [R], block_table [R, MB]) int32 on the device, reused while the requests'
        tables and lengths are unchanged (the device copy is never handed to callers).
        shared_rows: one request may also be served by its row of a batch's device copy (the
        row keeps the batch's MB columns), as when the reference's loop evicts requests one by
        one after one cal_attn over all of them; callers whose checks depend on MB leave it off.

        Entries are kept per stream: an upload is queued on the stream current at the time, so
        only work on that stream is ordered after it, and only that stream's later allocations
        can reuse the memory once the entry is dropped."""
        cur = self._stream_key()
        key = cur, tuple(reqs), tuple(ys) if ys is not None else None
        hit = self._dev_cache.get(key)
        tables, seq_used = self.tables, self.seq_used
        if hit is not None:
            # the entry holds the table objects themselves: identity, not id(), decides a hit,
            # then each table's mutation count, length and the request's length
            for r, t, (ver, n, s) in zip(reqs, hit[0], hit[1]):
                if tables[r] is not t or t.version != ver or len(t) != n or seq_used[r] != s:
                    break
            else:
                return hit[2], hit[3]
        if shared_rows and ys is None and len(reqs) == 1:
            r = reqs[0]
            t = tables[r]
            row_key = (cur, key[1], "row")   # apart from the request's own copy: its MB differs
            for ent, j, own in ((self._dev_cache.get(row_key), 0, True), (*self._batch_row(r, cur), False)):
                if ent is None:
                    continue
                ver, n, s = ent[1][j]
                if ent[0][j] is t and t.version == ver and len(t) == n and seq_used[r] == s:
                    if own:
                        return ent[2], ent[3]
                    seq, bt = ent[2][j:j + 1], ent[3][j:j + 1]
                    self._dev_cache[row_key] = ((t,), ((ver, n, s),), seq, bt)
                    return seq, bt
        host, mb = self._host_tables(reqs, ys)
        dev = self._upload(host)
        r_n = len(reqs)
        seq, bt = dev[:r_n], dev[r_n:].view(r_n, mb)
        tabs = tuple(self.tables[r] for r in reqs)
        if all(isinstance(t, _Table) for t in tabs):   # plain lists carry no mutation count
            if len(self._dev_cache) > 64:
                self._dev_cache.clear()
                self._dev_rows.clear()
            self._dev_cache[key] = (tabs, tuple((t.version, len(t), self.seq_used[r]) for t, r in zip(tabs, reqs)),
                                    seq, bt)
            if r_n > 1 and ys is None:
                for j, r in enumerate(reqs):
                    self._dev_rows[r] = (key, j)
        return seq, bt

    def _stream_key(self) -> int:
        """The current stream of the cache's device (0 on the CPU)."""
        dev = self._kv_dev
        return _hip.stream(dev) if dev.type == "cuda" else 0

    def _batch_row(self, r, cur):
        """(cache entry, row) of the last batch device copy that holds request r, uploaded on
        stream `cur`, or (None, 0)."""
        row = self._dev_rows.get(r)
        if row is None or row[0][0] != cur:
            return None, 0
        return self._dev_cache.get(row[0]), row[1]

    def _device_consts(self, values: tuple) -> torch.Tensor:
        """int32 device tensor holding `values`, shared by every call with the same values.
        Only for kernel inputs the kernels never write (budgets, protected counts): an
        eviction loop with fixed budgets then uploads nothing per call.  Kept per stream, as
        the device tables are."""
        key = (self._stream_key(), values)
        t = self._const_cache.get(key)
        if t is None:
            if len(self._const_cache) > 256:
                self._const_cache.clear()
            t = self._const_cache[key] = self._upload(np.array(values, dtype=np.int32))
        return t

    def block_table(self, reqs: list[int]) -> torch.Tensor:
        host, mb = self._host_tables(reqs)
        return self._upload(host[len(reqs):]).view(len(reqs), mb)

    def seq_tensor(self, reqs: list[int]) -> torch.Tensor:
        return self._upload(np.array([self.seq_used[r] for r in reqs], dtype=np.int32))

    def gather(self, req: int, layer: int = 0):
        slots = self.slot_map(req)
        flat = self.kv[layer].view(2, -1, self.n_kv_heads, self.head_dim)
        return flat[0, slots], flat[1, slots]

    # ---------------------------------------------------------------- primitives
    def decode_attention(self, reqs, q, layer=0, scale=None, *, n_valid=None, kv_len=None):
        """Paged attention -> (out, lse) on the GPU: the paged FlashAttention backend whose LSE
        by-product cal_attn consumes (the reference stands in for it with the torch
        paged_decode_attention_ref).  q [R, Hq, D] or [R, N, Hq, D]; layer=None attends every
        layer at once with q [L, R, N, Hq, D].  kv_len [R, N]: causal limits per query.
        Reference: actkv/paged.py:115-118."""
        kv = self.kv if layer is None else self.kv[layer]
        seq, bt = self._device_tables(reqs)
        return paged_decode_attention(q, kv, bt, seq, scale, n_valid=n_valid, kv_len=kv_len)

    def cal_attn(self, reqs, q, lse, out, n_seen, layer=0, scale=None, *, n_valid=None, kv_len=None):
        """Primitive 1: AttnScore <- CalAttn(target_q, KCache) via LSE recovery (Algorithm 3).

        layer=None scores every layer in one launch: q [L, R, N, Hq, D], lse [L, R, N, Hq],
        out [L, R, Hkv, W].  Reference: actkv/paged.py:120-123.
        """
        kv = self.kv if layer is None else self.kv[layer]
        seq, bt = self._device_tables(reqs)
        return action_scores(q, kv, bt, seq, lse, out, n_seen, scale, n_valid=n_valid, kv_len=kv_len)

    def _pinned_count(self, req: int, pinned: torch.Tensor) -> int:
        rec = self._pin_count.get(req)
        if rec is not None and rec[0] is pinned and rec[1] == pinned._version:
            return rec[2]
        cnt = int(pinned.sum())
        self._pin_count[req] = (pinned, pinned._version, cnt)
        return cnt

    def _compact_launch(self, reqs, bits, kept, pinned_in=None, pin_count=None, pin_out=None, *,
                        tables=None, flat=False):
        """One actkv_compact launch over `reqs` with packed keep bits [R, words] and host-known
        kept counts; then the host allocator updates in request order (sequential semantics).
        pinned_in [R, >=S] bool or pin_count [R] int32 (device) gives the pinned tokens;
        pin_out (optional, bool [R, >=max(kept)]) receives the survivors' pins.
        tables: the requests' (seq_used, block_table) device copies when the caller holds them.
        The kernel always reports each request's {B, M, drop, X} into a device buffer; with
        ACTKV_DEBUG=1 in the environment that report and the plan are read back and checked
        against the host's counts (one synchronisation per call).
        Returns perm [R, max(kept)] int64 and pinned_out [R, max(kept)] bool (or None); with
        flat=True and one request, perm [kept] and pinned_out [kept] (no per-request view)."""
        dev = self.kv.device
        bs = self.block_size
        r_n = len(reqs)
        seqs = [self.seq_used[r] for r in reqs]
        ys = [-(-s // bs) for s in seqs]
        seq_dev, bt_dev = self._device_tables(reqs) if tables is None else tables
        mb = bt_dev.shape[1]
        bmax = max(max(kept), 1)
        flat = flat and r_n == 1 and pin_out is None
        shape = (bmax,) if flat else (r_n, bmax)
        perm = torch.empty(shape, dtype=torch.int64, device=dev)
        if pin_out is None and (pinned_in is not None or pin_count is not None):
            pin_out = torch.empty(shape, dtype=torch.bool, device=dev)
        counts = _hip.scratch(dev, "compact_counts", 16 * r_n)
        debug = _hip.debug()
        if debug:
            smax = max(max(seqs), 1)
            src = torch.full((r_n, smax), -1, dtype=torch.int64, device=dev)
            dst = torch.full((r_n, smax), -1, dtype=torch.int64, device=dev)
        es = self.kv.element_size()
        row = self.n_kv_heads * self.head_dim
        if self.kv.is_contiguous():     # [L*2 planes, NB*BS slots, row] from the cache's own strides
            kvs = self.kv.stride()
            planes, plane_b, slot_b = self.n_layers * 2, kvs[1] * es, kvs[3] * es
        else:
            flat = self.kv.view(self.n_layers * 2, -1, row)
            planes, plane_b, slot_b = flat.shape[0], flat.stride(0) * es, flat.stride(1) * es
        rc = _hip.glue().compact(
            self.kv.data_ptr(), planes, plane_b, slot_b, row * es, self.num_blocks,
            bits.data_ptr(), bits.stride(0), r_n, seq_dev.data_ptr(),
            bt_dev.data_ptr(), mb, bs,
            perm.data_ptr(), bmax, _hip.ptr(pinned_in), 0 if pinned_in is None else pinned_in.stride(0),
            _hip.ptr(pin_count), _hip.ptr(pin_out), bmax if pin_out is None or flat else pin_out.stride(0),
            None, 0, None, 0, _hip.ptr(src) if debug else None, _hip.ptr(dst) if debug else None,
            src.shape[1] if debug else 0, counts.data_ptr(),
            1, max(seqs), max(kept), _hip.stream(dev))
        _hip.check(rc, "actkv_compact")
        if debug:
            _check_compaction(reqs, seqs, kept, bs, bits, counts.view(torch.int32)[: 4 * r_n].view(r_n, 4),
                              src, dst)
        for i, r in enumerate(reqs):
            drop = ys[i] - -(-kept[i] // bs)
            table = self.tables[r]
            if drop > 0:                      # freed blocks pushed last-first: table[drop-1], ..., table[0]
                self.free.extend(table[drop - 1::-1])
            self.tables[r] = table.tail(drop) if isinstance(table, _Table) else table[drop:]
            self.seq_used[r] = kept[i]
        if flat and kept[0] < bmax:     # nothing kept: empty results
            return perm[:0], None if pin_out is None else pin_out[:0]
        return perm, pin_out

    def compact(self, req: int, keep_mask: torch.Tensor) -> torch.Tensor:
        """Primitive 3: KVCache <- Compaction(KVCache, KeepMask) (Algorithm 4), all layers at once.

        Returns `perm` (new logical position -> old logical position) so callers can permute
        per-token metadata.  Freed blocks go straight back to the allocator.
        Reference: actkv/paged.py:125-139.
        """
        dev = _hip.require_gpu("PagedKVCache.compact", self.kv, keep_mask)
        n = self.seq_used[req]
        keep = keep_mask[:n]
        if keep.dtype != torch.bool:
            keep = keep.bool()
        keep = keep.contiguous()
        seq = upload_i32([n], dev)
        bits = torch.empty(1, max(keep_words(n, self.block_size), 1), dtype=torch.int32, device=dev)
        kept = torch.empty(1, dtype=torch.int32, device=dev)
        _hip.check(_hip.lib().actkv_pack_keep(keep.data_ptr(), keep.numel(), 1, seq.data_ptr(), self.block_size,
                                              bits.data_ptr(), bits.shape[1], kept.data_ptr(), n,
                                              _hip.stream(dev)), "actkv_pack_keep")
        b = int(kept.item())    # the one synchronisation: B sizes perm and the host lists
        perm, _ = self._compact_launch([req], bits, [b])
        return perm[0, :b]

    def evict(self, req: int, scores: torch.Tensor, budget: int, protected: int = 0,
              head_reduce: str = "mean") -> torch.Tensor:
        """Scores -> KeepMask -> Compaction: keep the protected prefix plus the top-`budget` tokens.

        `protected` counts the request's first tokens (e.g. the prompt) the first time it is evicted.
        Compaction moves them, so the cache remembers where they went and keeps protecting them.
        Returns `perm` like compact(); a request already within budget is left untouched.
        Reference: actkv/paged.py:141-157.
        """
        return self.evict_batch([req], [scores], budget, protected, head_reduce)[0]

    def evict_batch(self, reqs: list[int], scores, budget, protected=0,
                    head_reduce: str = "mean") -> list[torch.Tensor]:
        """`evict` for several requests with one keep-mask launch and one compaction launch.

        Equal to calling evict(reqs[i], scores[i], budget[i], protected[i]) in order (the free
        list ends in the same order).  scores: a list with one [S]/[Hkv, S]/[L, Hkv, S] tensor
        per request, or one tensor [..., R, Hkv, W] (leading dims are layers), e.g. the
        [L, R, Hkv, W] output of a multi-layer cal_attn.  budget / protected: an int for every
        request or one per request.  Each request may appear once (ValueError otherwise).
        head_reduce is checked once a request is over its budget (ValueError), as the
        reference checks it in keep_mask_from_scores after the within-budget return.
        """
        reqs = list(reqs)
        if len(set(reqs)) != len(reqs):
            raise ValueError("evict_batch: each request once")
        r_n = len(reqs)
        budgets = list(budget) if isinstance(budget, (list, tuple)) else [budget] * r_n
        prots = list(protected) if isinstance(protected, (list, tuple)) else [protected] * r_n
        dev = self.kv.device
        out = [None] * r_n
        active, pinneds, kept, counts = [], [], [], []
        for i, req in enumerate(reqs):
            n = self.seq_used[req]
            pinned = self.pinned.get(req)
            if pinned is None:
                # first eviction: the protected prefix is a count; the kernels build the
                # mask of the survivors themselves (no device mask needed beforehand)
                cnt = min(max(int(prots[i]), 0), n)
                if n - cnt <= budgets[i]:
                    pinned = torch.arange(n, device=dev) < prots[i]
                    self.pinned[req] = pinned
                    self._pin_count[req] = (pinned, pinned._version, cnt)
                    out[i] = torch.arange(n, device=dev)
                    continue
                active.append(i)
                pinneds.append(None)
                kept.append(cnt + max(budgets[i], 0))
                counts.append(cnt)
                continue
            if pinned.numel() > n:
                # the reference's torch.cat with a negative-size pad raises here (paged.py:151)
                raise RuntimeError(f"evict: request {req} has {pinned.numel()} pinned flags for {n} tokens "
                                   "(a compact() since the last evict() left them unmapped)")
            cnt = self._pinned_count(req, pinned)
            if pinned.numel() < n:                      # tokens appended since
                pinned = torch.cat([pinned, pinned.new_zeros(n - pinned.numel())])
                self._pin_count[req] = (pinned, pinned._version, cnt)
            self.pinned[req] = pinned
            if n - cnt <= budgets[i]:
                out[i] = torch.arange(n, device=dev)
                continue
            active.append(i)
            pinneds.append(pinned)
            kept.append(cnt + max(budgets[i], 0))
            counts.append(cnt)
        if not active:
            return out
        if head_reduce not in _REDUCE:
            raise ValueError(head_reduce)
        _hip.require_gpu("PagedKVCache.evict", self.kv)
        a_reqs = [reqs[i] for i in active]
        seqs = [self.seq_used[r] for r in a_reqs]
        smax = max(seqs)
        ra = len(active)
        # scores -> (tensor, L, H, layer / request / head strides), read in place where possible
        if isinstance(scores, torch.Tensor):
            _hip.require_gpu("PagedKVCache.evict", scores)
            if scores.dim() < 3:
                raise ValueError("a scores tensor for several requests is [..., R, Hkv, W]")
            sc = scores
            if sc.shape[-3] != r_n:
                raise ValueError(f"scores {tuple(scores.shape)} do not have {r_n} requests at dim -3")
            sc = sc.reshape(-1, *sc.shape[-3:]) if sc.dim() != 4 else sc
            sc = sc[:, active] if ra != r_n else sc
            if sc.shape[-1] < smax:
                raise ValueError(f"scores cover {sc.shape[-1]} tokens, a request holds {smax}")
            if sc.dtype not in _SCORE_DTYPES:
                sc = sc.float()
            if sc.stride(-1) != 1:
                sc = sc.contiguous()
            L, _, H, _ = sc.shape
            s_sl, s_sr, s_sh, _ = sc.stride()
        elif ra == 1:
            s_i = scores[active[0]]
            _hip.require_gpu("PagedKVCache.evict", s_i)
            sc, L, H, s_sl, s_sh = _scores_layout(s_i, seqs[0])
            s_sr = 0
        else:
            per = []
            for i in active:
                s_i = scores[i]
                _hip.require_gpu("PagedKVCache.evict", s_i)
                s3, L_i, H_i, _, _ = _scores_layout(s_i, self.seq_used[reqs[i]])
                per.append(s3.reshape(L_i, H_i, -1))
            L, H = per[0].shape[0], per[0].shape[1]
            if any(p.shape[0] != L or p.shape[1] != H for p in per):
                raise ValueError("every request's scores need the same layer and head counts")
            sc = torch.zeros(L, ra, H, smax, dtype=per[0].dtype, device=dev)
            for j, p in enumerate(per):
                sc[:, j, :, : seqs[j]] = p[..., : seqs[j]]
            s_sl, s_sr, s_sh, _ = sc.stride()
        # the lengths come with the block tables the compaction launch reads anyway; budgets and
        # protected counts are the same from call to call in an eviction loop
        tables = self._device_tables(a_reqs, shared_rows=True)
        consts = self._device_consts(tuple(max(budgets[i], 0) for i in active) + tuple(counts))
        if all(p is None for p in pinneds):           # every request's pins are a prefix count
            pin_mat, prot_count = None, consts[ra:]
        else:
            prot_count = None
            if ra == 1:
                pin_mat = pinneds[0].view(1, -1)
            else:
                pin_mat = torch.zeros(ra, smax, dtype=torch.bool, device=dev)
                for j, p in enumerate(pinneds):
                    if p is None:
                        pin_mat[j, : counts[j]] = True
                    else:
                        pin_mat[j, : p.numel()] = p
        _, bits = _keep_mask_launch(sc, L, H, s_sl, s_sr, s_sh, ra,
                                    tables[0], consts[:ra], prot_count, pin_mat,
                                    0 if pin_mat is None else pin_mat.stride(0),
                                    head_reduce, self.block_size, smax, dev, want_keep=False)
        perm, pin_out = self._compact_launch(a_reqs, bits, kept, pin_mat, prot_count, tables=tables,
                                             flat=True)
        if ra == 1:                                   # flat results: no per-request views
            i = active[0]
            out[i] = perm
            self.pinned[reqs[i]] = pin_out
            self._pin_count[reqs[i]] = (pin_out, pin_out._version, counts[0])
            return out
        for j, i in enumerate(active):
            b = kept[j]
            out[i] = perm[j, :b]
            newpin = pin_out[j, :b]
            self.pinned[reqs[i]] = newpin
            self._pin_count[reqs[i]] = (newpin, newpin._version, counts[j])
        return out
