"""CPU restatement of the ActKV eviction path (test infrastructure; see oracle/__init__.py).

Float work follows the reference's torch float32 semantics on the CPU; integer and byte work
(compaction planning, row moves, allocator) is numpy.  Each function cites the reference
lines it restates (paths relative to the reference repository).
"""
from __future__ import annotations

import math

import numpy as np
import torch

# ============================================================================ scoring

def gather_k(kv_layer: torch.Tensor, table_row, seq_used: int) -> torch.Tensor:
    """K rows [S, Hkv, D] of one request in logical order (lse_attn.py:32-39)."""
    bs = kv_layer.shape[2]
    nblk = -(-seq_used // bs)
    blocks = torch.as_tensor(np.asarray(table_row[:nblk], dtype=np.int64))
    return kv_layer[0].index_select(0, blocks).reshape(-1, kv_layer.shape[3], kv_layer.shape[4])[:seq_used]


def decode_lse(q: torch.Tensor, kv_layer: torch.Tensor, table, seq_used, scale=None,
               dtype=torch.float64) -> torch.Tensor:
    """lse[r, h] = logsumexp_t scale * q[r,h] . k[t, h // G] over all seq_used tokens
    (lse_attn.py:42-60, the by-product Algorithm 3 consumes).  q [R, Hq, D] -> [R, Hq] float32,
    accumulated in `dtype`."""
    r_n, hq, d = q.shape
    hkv = kv_layer.shape[3]
    g = hq // hkv
    scale = d ** -0.5 if scale is None else scale
    lse = torch.empty(r_n, hq, dtype=torch.float32)
    for r in range(r_n):
        s = int(seq_used[r])
        k = gather_k(kv_layer, table[r], s).to(dtype)                 # [S, Hkv, D]
        qq = q[r].to(dtype).view(hkv, g, d)
        logits = torch.einsum("hgd,shd->hgs", qq, k) * scale        # [Hkv, G, S]
        lse[r] = torch.logsumexp(logits, -1).reshape(hq).float()
    return lse


def gather_v(kv_layer: torch.Tensor, table_row, seq_used: int) -> torch.Tensor:
    """V rows [S, Hkv, D] of one request in logical order (lse_attn.py:32-40)."""
    bs = kv_layer.shape[2]
    nblk = -(-seq_used // bs)
    blocks = torch.as_tensor(np.asarray(table_row[:nblk], dtype=np.int64))
    return kv_layer[1].index_select(0, blocks).reshape(-1, kv_layer.shape[3], kv_layer.shape[4])[:seq_used]


def paged_attention(q: torch.Tensor, kv_layer: torch.Tensor, table, seq_used, scale=None, kv_len=None,
                    n_valid=None, dtype=torch.float64):
    """(out [R, N, Hq, D], lse [R, N, Hq]) float32 of paged attention, accumulated in `dtype`.

    Restates paged_decode_attention_ref (lse_attn.py:42-60): per request, gather K and V, repeat
    the KV heads over the GQA group, logits = scale * q . k, lse = logsumexp(logits), out =
    softmax(logits) @ v.  Additive, as the device entry point: N queries per request (q
    [R, N, Hq, D]), kv_len [R, N] (query n sees tokens t < kv_len[r][n], clamped to seq_used) and
    n_valid [R] (rows n >= n_valid[r] stay 0).  A query that sees no token gets lse = -inf and
    out = 0 (torch's logsumexp and softmax-einsum over an empty set)."""
    r_n, n_q, hq, d = q.shape
    hkv = kv_layer.shape[3]
    g = hq // hkv
    scale = d ** -0.5 if scale is None else scale
    out = torch.zeros(r_n, n_q, hq, d, dtype=torch.float32)
    lse = torch.zeros(r_n, n_q, hq, dtype=torch.float32)
    for r in range(r_n):
        s = int(seq_used[r])
        k = gather_k(kv_layer, table[r], s).to(dtype).repeat_interleave(g, dim=1)   # [S, Hq, D]
        v = gather_v(kv_layer, table[r], s).to(dtype).repeat_interleave(g, dim=1)
        nv = n_q if n_valid is None else min(max(int(n_valid[r]), 0), n_q)
        for n in range(nv):
            lim = s if kv_len is None else min(max(int(kv_len[r][n]), 0), s)
            if lim == 0:
                lse[r, n] = -math.inf
                continue
            logits = torch.einsum("hd,shd->hs", q[r, n].to(dtype), k[:lim]) * scale     # [Hq, lim]
            lse[r, n] = torch.logsumexp(logits, -1).float()
            out[r, n] = torch.einsum("hs,shd->hd", torch.softmax(logits, -1), v[:lim]).float()
    return out, lse


def _group_probs(q_r: torch.Tensor, k: torch.Tensor, lse_r: torch.Tensor, scale: float) -> torch.Tensor:
    """max over the GQA group of exp(scale * q.k - lse): q_r [Hq, D], k [S, Hkv, D] -> [Hkv, S]
    (lse_attn.py:68-72: max over the group first, float32)."""
    hkv = k.shape[1]
    g = q_r.shape[0] // hkv
    kk = k.float().repeat_interleave(g, dim=1)                       # [S, Hq, D]
    logits = torch.einsum("hd,shd->hs", q_r.float(), kk) * scale      # [Hq, S]
    p = torch.exp(logits - lse_r.unsqueeze(-1))
    return p.view(hkv, g, -1).amax(1)


def action_scores_fold(q, kv_layer, table, seq_used, lse, out, n_seen, scale=None):
    """ONE action query per request folded into the running mean (lse_attn.py:63-78):
    out[r, :, :S] += (p - out[r, :, :S]) / (n_seen[r] + 1); then n_seen += 1.
    q [R, Hq, D], lse [R, Hq] float32, out [R, Hkv, W] float32 (in place), n_seen [R] int32."""
    d = q.shape[-1]
    scale = d ** -0.5 if scale is None else scale
    for r in range(q.shape[0]):
        s = int(seq_used[r])
        p = _group_probs(q[r], gather_k(kv_layer, table[r], s), lse[r], scale)
        cur = out[r, :, :s]
        out[r, :, :s] = cur + (p - cur) / (float(n_seen[r]) + 1.0)
    n_seen += 1
    return out


def action_scores_nfold(q, kv_layer, table, seq_used, lse, out, n_seen, scale=None,
                        n_valid=None, kv_len=None):
    """N action queries per request: N successive action_scores_fold folds, with the q.k
    products of all N queries batched per KV head (equal to the one-at-a-time folds up to
    float32 dot-product rounding).
    q [R, N, Hq, D], lse [R, N, Hq]; n_valid [R] (queries folded per request) and kv_len
    [R, N] (query n sees tokens t < kv_len[r, n]; unseen tokens contribute 0)."""
    r_n, n_q, hq, d = q.shape
    hkv = kv_layer.shape[3]
    g = hq // hkv
    scale = d ** -0.5 if scale is None else scale
    for r in range(r_n):
        s = int(seq_used[r])
        nq = n_q if n_valid is None else max(0, min(int(n_valid[r]), n_q))
        k = gather_k(kv_layer, table[r], s).float()                   # [S, Hkv, D]
        cur = out[r, :, :s].clone()
        n0 = float(n_seen[r])
        probs = torch.empty(nq, hkv, s)
        for h in range(hkv):
            qh = q[r, :nq, h * g:(h + 1) * g].float()                  # [nq, G, D]
            logits = torch.einsum("ngd,sd->ngs", qh, k[:, h]) * scale
            p = torch.exp(logits - lse[r, :nq, h * g:(h + 1) * g].unsqueeze(-1))
            probs[:, h] = p.amax(1)
        if kv_len is not None:
            t = torch.arange(s)
            for n in range(nq):
                probs[n, :, t >= int(kv_len[r, n])] = 0.0
        for n in range(nq):
            cur = cur + (probs[n] - cur) / (n0 + n + 1.0)
        out[r, :, :s] = cur
        n_seen[r] += nq
    return out


# ============================================================================ keep mask

def keep_mask_from_scores(scores: torch.Tensor, seq_used: int, budget: int, protected=0,
                          head_reduce: str = "mean") -> torch.Tensor:
    """Protected tokens + the top-`budget` others by the layer-averaged head-reduced score
    (paged.py:23-46), with torch CPU float32 reductions and torch.topk."""
    if head_reduce not in ("mean", "max"):
        raise ValueError(head_reduce)
    x = scores[..., :seq_used].float()
    if x.dim() >= 2:
        x = x.amax(-2) if head_reduce == "max" else x.mean(-2)
        x = x.reshape(-1, seq_used).mean(0)
    if isinstance(protected, torch.Tensor):
        keep = protected.to(dtype=torch.bool).clone()
    else:
        keep = torch.arange(seq_used) < protected
    cand = torch.nonzero(~keep).flatten()
    k = min(budget, cand.numel())
    if k > 0:
        keep[cand[torch.topk(x[cand], k).indices]] = True
    return keep


def reduced_scores(scores: torch.Tensor, seq_used: int, head_reduce: str = "mean") -> torch.Tensor:
    """The per-token score keep_mask_from_scores ranks (paged.py:34-37)."""
    x = scores[..., :seq_used].float()
    if x.dim() >= 2:
        x = x.amax(-2) if head_reduce == "max" else x.mean(-2)
        x = x.reshape(-1, seq_used).mean(0)
    return x


def keep_mask_lowest_index_ties(scores, seq_used, budget, protected=0, head_reduce="mean"):
    """keep_mask_from_scores with a defined tie rule: among equal scores the lower index is
    taken first (a stable descending sort).  torch.topk leaves that order unspecified; the
    two agree whenever the k-th and (k+1)-th candidate scores differ."""
    x = reduced_scores(scores, seq_used, head_reduce)
    if isinstance(protected, torch.Tensor):
        keep = protected.to(dtype=torch.bool).clone()
    else:
        keep = torch.arange(seq_used) < protected
    cand = torch.nonzero(~keep).flatten()
    k = min(budget, cand.numel())
    if k > 0:
        order = torch.sort(x[cand], descending=True, stable=True).indices
        keep[cand[order[:k]]] = True
    return keep


def _cascade(rows: np.ndarray) -> np.ndarray:
    """float32 column sums of rows [n, cols] in the order of torch's CPU multi_row_sum
    (16-row blocks, 4 accumulator levels)."""
    f32 = np.float32
    n = rows.shape[0]
    acc = [np.zeros(rows.shape[1:], f32) for _ in range(4)]
    i = 0
    while i + 16 <= n:
        for j in range(16):
            acc[0] = (acc[0] + rows[i + j]).astype(f32)
        i += 16
        for lev in range(1, 4):
            acc[lev] = (acc[lev] + acc[lev - 1]).astype(f32)
            acc[lev - 1] = np.zeros_like(acc[0])
            if i & (15 << (4 * lev)):
                break
    while i < n:
        acc[0] = (acc[0] + rows[i]).astype(f32)
        i += 1
    for lev in range(1, 4):
        acc[0] = (acc[0] + acc[lev]).astype(f32)
    return acc[0]


def _ilp4(rows: np.ndarray) -> np.ndarray:
    """torch's CPU row_sum order: 4 interleaved cascades, leftovers into the first."""
    f32 = np.float32
    n = rows.shape[0]
    m = n // 4
    parts = [_cascade(rows[k:4 * m:4]) if m else np.zeros(rows.shape[1:], f32) for k in range(4)]
    for i in range(4 * m, n):
        parts[0] = (parts[0] + rows[i]).astype(f32)
    out = parts[0]
    for k in range(1, 4):
        out = (out + parts[k]).astype(f32)
    return out


def torch_mean_emulation(rows: np.ndarray, n_cols: int) -> np.ndarray:
    """mean over axis 0 of float32 rows [n, n_cols] as torch's CPU kernel computes it: the
    32-column-aligned body in cascade order, the last n_cols % 32 columns in row_sum order,
    then an IEEE division by n.  This is the order the device keep-mask reduction follows."""
    rows = np.asarray(rows, dtype=np.float32)
    n = rows.shape[0]
    body = n_cols - n_cols % 32
    out = np.empty(n_cols, np.float32)
    out[:body] = _cascade(rows[:, :body])
    if body < n_cols:
        out[body:] = _ilp4(rows[:, body:])
    return (out / np.float32(n)).astype(np.float32)


# ============================================================================ compaction

def plan_compaction(keep_mask, seq_used: int, table_row, block_size: int):
    """Algorithm 4 steps 1-5 (compaction.py:44-69): returns (src_slots, dst_slots, perm, drop)
    as int64 numpy arrays (physical slots, new->old logical) and the dropped block count."""
    keep = np.asarray(keep_mask[:seq_used], dtype=bool)
    table = np.asarray(table_row, dtype=np.int64)
    b = int(keep.sum())
    y = -(-seq_used // block_size)
    x = -(-b // block_size)
    start = (y - x) * block_size
    end = start + b
    full = np.zeros(y * block_size, dtype=bool)
    full[:seq_used] = keep
    dst = np.flatnonzero(~full[start:end]) + start
    outside = full.copy()
    outside[start:end] = False
    src = np.flatnonzero(outside)
    assert src.size == dst.size
    perm = np.arange(start, end, dtype=np.int64)
    perm[dst - start] = src

    def phys(l):
        return table[l // block_size] * block_size + l % block_size

    return phys(src), phys(dst), perm, y - x


def plan_compaction_bruteforce(keep_mask, seq_used: int, table_row, block_size: int):
    """The same plan from the definition with plain Python loops (small inputs only)."""
    keep = [bool(keep_mask[i]) for i in range(seq_used)]
    b = sum(keep)
    y = (seq_used + block_size - 1) // block_size
    x = (b + block_size - 1) // block_size
    start = (y - x) * block_size
    end = start + b
    kept_at = lambda l: l < seq_used and keep[l]
    holes = [l for l in range(start, end) if not kept_at(l)]
    movers = [l for l in range(y * block_size) if (l < start or l >= end) and kept_at(l)]
    perm = list(range(start, end))
    for s, d in zip(movers, holes):
        perm[d - start] = s
    phys = lambda l: int(table_row[l // block_size]) * block_size + l % block_size
    return [phys(l) for l in movers], [phys(l) for l in holes], perm, y - x


def apply_copies(kv_flat: np.ndarray, src, dst) -> None:
    """kv_flat[p, dst[i]] = kv_flat[p, src[i]] for every plane (compaction.py:72-74); any dtype,
    byte-exact."""
    src = np.asarray(src, dtype=np.int64)
    dst = np.asarray(dst, dtype=np.int64)
    if src.size:
        kv_flat[:, dst] = kv_flat[:, src]


# ============================================================================ paged cache

class PagedCacheModel:
    """The reference PagedKVCache (paged.py:49-157) on the CPU with numpy storage.

    kv holds raw element bits ([L, 2, NB, BS, Hkv, D], e.g. uint16 for bf16/fp16 caches), so
    compaction is byte-exact; `free` is a stack (pop from the end), freed blocks are pushed
    in reverse so the first freed block is allocated next (paged.py:56, :73-74, :135-137)."""

    def __init__(self, num_blocks, block_size, n_kv_heads, head_dim, n_layers=1, np_dtype=np.uint16):
        self.num_blocks, self.block_size = num_blocks, block_size
        self.n_kv_heads, self.head_dim, self.n_layers = n_kv_heads, head_dim, n_layers
        self.kv = np.zeros((n_layers, 2, num_blocks, block_size, n_kv_heads, head_dim), dtype=np_dtype)
        self.free = list(range(num_blocks - 1, -1, -1))
        self.tables: dict[int, list[int]] = {}
        self.seq_used: dict[int, int] = {}
        self.pinned: dict[int, np.ndarray] = {}

    @property
    def used_blocks(self):
        return self.num_blocks - len(self.free)

    def append(self, req, k, v):
        """k, v: [n_layers, n, Hkv, D] arrays of the storage dtype (paged.py:67-85)."""
        n = k.shape[1]
        start = self.seq_used.get(req, 0)
        table = self.tables.setdefault(req, [])
        self.seq_used.setdefault(req, 0)
        need = -(-(start + n) // self.block_size) - len(table)
        if need > len(self.free):
            raise RuntimeError(f"need {need} blocks, {len(self.free)} free")
        for _ in range(need):
            table.append(self.free.pop())
        flat = self.kv.reshape(self.n_layers, 2, -1, self.n_kv_heads, self.head_dim)
        slots = self.slot_map(req, start + n)[start:]
        flat[:, 0, slots] = k
        flat[:, 1, slots] = v
        self.seq_used[req] = start + n

    def slot_map(self, req, n=None):
        n = self.seq_used[req] if n is None else n
        pos = np.arange(n)
        return np.asarray(self.tables[req], dtype=np.int64)[pos // self.block_size] * self.block_size + pos % self.block_size

    def gather(self, req, layer=0):
        flat = self.kv[layer].reshape(2, -1, self.n_kv_heads, self.head_dim)
        s = self.slot_map(req)
        return flat[0, s], flat[1, s]

    def compact(self, req, keep_mask):
        """paged.py:125-139: plan, move every layer's K and V rows, reclaim the leading blocks."""
        src, dst, perm, drop = plan_compaction(keep_mask, self.seq_used[req], self.tables[req], self.block_size)
        flat = self.kv.reshape(self.n_layers * 2, -1, self.n_kv_heads * self.head_dim)
        apply_copies(flat, src, dst)
        freed = self.tables[req][:drop]
        self.tables[req] = self.tables[req][drop:]
        self.free.extend(reversed(freed))
        self.seq_used[req] = int(perm.size)
        return perm

    def evict(self, req, scores, budget, protected=0, head_reduce="mean", tie_rule="torch"):
        """paged.py:141-157 (pinned prefix remembered across evictions).  tie_rule "lowest"
        uses keep_mask_lowest_index_ties instead of torch.topk's unspecified tie order."""
        n = self.seq_used[req]
        pinned = self.pinned.get(req)
        if pinned is None:
            pinned = np.arange(n) < protected
        if pinned.size < n:
            pinned = np.concatenate([pinned, np.zeros(n - pinned.size, dtype=bool)])
        self.pinned[req] = pinned
        if n - int(pinned.sum()) <= budget:
            return np.arange(n)
        fn = keep_mask_lowest_index_ties if tie_rule == "lowest" else keep_mask_from_scores
        keep = fn(scores, n, budget, torch.from_numpy(pinned.copy()), head_reduce).numpy()
        perm = self.compact(req, keep)
        self.pinned[req] = pinned[perm]
        return perm


# ============================================================================ LRFU keep score

def top_p_mask(scores: torch.Tensor, p: float, stable: bool = False, total64: bool = False) -> torch.Tensor:
    """Nucleus mask (eviction.py:36-50): the smallest set of entries, taken in descending order,
    whose cumulative sum reaches p * total, restricted to positive entries.  torch CPU
    semantics: float32 total, float32 threshold p * total, cumsum accumulated in float64 and
    stored as float32, left searchsorted.  stable=False sorts exactly as the reference (torch's
    default sort, whose order among equal scores is unspecified); stable=True takes equal
    scores lower index first, the rule the device kernel follows.  total64=True rounds the
    float64 total to float32 (the device kernel's total) instead of torch's float32
    summation order, which depends on the host's SIMD width; the two totals differ by a few
    ulps, which moves the nucleus boundary only when a running sum lies that close to it."""
    if scores.numel() == 0:
        return torch.zeros_like(scores, dtype=torch.bool)
    total = scores.double().sum().float() if total64 else scores.sum()
    if total <= 0:
        return torch.zeros_like(scores, dtype=torch.bool)
    vals, order = torch.sort(scores, descending=True, stable=stable)
    csum = torch.cumsum(vals, 0)
    n_keep = int(torch.searchsorted(csum, p * total).item()) + 1
    n_keep = min(n_keep, scores.numel())
    mask = torch.zeros_like(scores, dtype=torch.bool)
    mask[order[:n_keep]] = True
    return mask & (scores > 0)


def top_p_mask_bruteforce(scores, p: float):
    """The nucleus from its definition with Python loops and float64 sums (small inputs):
    walk the entries in descending order (ties: lower index first) until the running sum
    reaches p * total; keep those entries that are positive."""
    vals = [float(x) for x in scores]
    total = sum(vals)
    if not vals or total <= 0:
        return [False] * len(vals)
    order = sorted(range(len(vals)), key=lambda i: (-vals[i], i))
    keep = [False] * len(vals)
    run = 0.0
    for i in order:
        keep[i] = vals[i] > 0
        run += vals[i]
        if run >= p * total:
            break
    return keep


def lrfu_update(ks: torch.Tensor, act: torch.Tensor, seq_used: int, protected: int, decay: float,
                top_p: float, active: bool = True, stable: bool = False):
    """Algorithm 1 steps 2-4 for one layer row (eviction.py:209-218): over entries
    [protected, seq_used), hit = top_p_mask(act) (none when the round had no action tokens),
    ks = decay * ks, then ks[hit] += act[hit].  ks, act: float32 [>= seq_used], ks in place.
    Returns the hit mask over [protected, seq_used)."""
    a = act[protected:seq_used]
    hit = top_p_mask(a, top_p, stable) if active else torch.zeros_like(a, dtype=torch.bool)
    k = ks[protected:seq_used]
    k.mul_(decay)
    k[hit] += a[hit]
    return hit


def paged_lrfu_act(scores: torch.Tensor, seq_used: int, head_reduce: str = "mean") -> torch.Tensor:
    """Per-layer, per-token action score of the paged cache: the action-region scores
    [L, Hkv, W] (running mean over the round's action queries of the GQA-group max,
    lse_attn.py:63-78) reduced over KV heads (eviction.py:20-33) -> [L, seq_used] float32."""
    x = scores[..., :seq_used].float()
    return x.amax(-2) if head_reduce == "max" else x.mean(-2)


def paged_lrfu_update(ks: torch.Tensor, act: torch.Tensor, seq_used: int, pinned, decay: float,
                      top_p: float, active: bool = True, stable: bool = True,
                      total64: bool = False) -> torch.Tensor:
    """lrfu_update for every layer of one request of the paged cache: ks [L, >=S] (in place),
    act [L, >=S].  `pinned` is a prefix count or a bool mask [>=S] of protected tokens; the
    nucleus runs over the other tokens in index order (a prefix count gives exactly
    eviction.py:209-218's act[layer, protected:]).  Returns hits [L, S] bool."""
    S = seq_used
    if isinstance(pinned, torch.Tensor):
        free = torch.nonzero(~pinned[:S].bool()).flatten()
    else:
        free = torch.arange(min(max(int(pinned), 0), S), S)
    hits = torch.zeros(ks.shape[0], S, dtype=torch.bool)
    for l in range(ks.shape[0]):
        a = act[l, free]
        hit = top_p_mask(a, top_p, stable, total64) if active else torch.zeros_like(a, dtype=torch.bool)
        k = ks[l, free] * decay
        k[hit] += a[hit]
        ks[l, free] = k
        hits[l, free] = hit
    return hits
