"""Recovery-based attention scoring on a paged KV cache (ActKV Algorithm 3), on gfx950.

Drop-in for the reference module actkv/kernels/lse_attn.py: same names, arguments, in-place
semantics and errors.  `action_scores` runs the HIP kernels of libactkv_hip.so (bf16/fp16
MFMA kernels for head_dim 128 or 64 and 1 to 16 query heads per KV head; a VALU kernel for
every other shape and for float32 caches).  It has no CPU path: CPU tensors raise.

Layout (vLLM-style), one layer:
    kv          [2, num_blocks, block_size, n_kv_heads, head_dim]
    block_table [R, max_blocks] int32, logical block -> physical block
    seq_used    [R] int32, valid tokens per request
Output, updated in place:
    out         [R, n_kv_heads, max_blocks * block_size] float32, running mean over action tokens
    n_seen      [R] int32, action tokens already folded into `out` for each request

Additive extensions (they reduce to the reference for one query and one layer):
    q [R, N, Hq, D] with lse [R, N, Hq] folds N action tokens in one launch, and
    q [L, R, N, Hq, D], kv [L, 2, NB, BS, Hkv, D], lse [L, R, N, Hq], out [L, R, Hkv, W]
    score every layer in that same launch (n_seen counts action tokens, not layers).
    n_valid [R] int32: request r folds only its first n_valid[r] of the N queries.
    kv_len [R, N] int32: query n of request r sees only tokens t < kv_len[r, n] (causal
    action region); tokens it cannot see contribute probability 0.

`gather_kv`, `paged_decode_attention_ref` and `action_scores_ref` are the reference's torch
formulations (lse_attn.py:32-78), kept so callers of the reference module find them; the
HIP path never calls them.
"""
from __future__ import annotations

import math

import torch

from .. import _hip

HAS_KERNELS = _hip.available()
# The reference's flag for "compiled kernels are active" (tests and the bench read it).
HAS_TRITON = HAS_KERNELS


# ----------------------------------------------------------------------------- reference (torch)

def gather_kv(kv: torch.Tensor, block_table: torch.Tensor, seq_used: int, row: int):
    """Contiguous K, V [S, H, D] for one request (what a gather-based approach materializes).

    Token t of the request sits in slot block_table[row, t // bs] * bs + t % bs of either
    plane.  Reference: actkv/kernels/lse_attn.py:32-39.
    """
    bs = kv.shape[2]
    t = torch.arange(seq_used, device=kv.device)
    slots = block_table[row].to(device=kv.device, dtype=torch.long)[t // bs] * bs + t % bs
    planes = kv.reshape(2, -1, kv.shape[3], kv.shape[4])
    return planes[0].index_select(0, slots), planes[1].index_select(0, slots)


def _group_logits(q_r: torch.Tensor, k: torch.Tensor, scale: float) -> torch.Tensor:
    """scale * q . k for one request, grouped by KV head: q_r [Hq, D], k [S, Hkv, D] ->
    [Hkv, G, S] float32 (query head h*G + g reads KV head h)."""
    hkv = k.shape[1]
    qg = q_r.float().reshape(hkv, -1, q_r.shape[-1])                 # [Hkv, G, D]
    return torch.matmul(qg, k.float().permute(1, 2, 0)) * scale      # [Hkv, G, S]


def paged_decode_attention_ref(q, kv, block_table, seq_used, scale=None):
    """Plain decode attention over a paged cache. Returns (out [R,Hq,D], lse [R,Hq]), float32.

    lse[r, h] = logsumexp_t scale * q[r, h] . k_t and out = softmax @ V over the request's
    tokens.  Reference: actkv/kernels/lse_attn.py:42-60 (stands in for the paged
    FlashAttention backend whose LSE by-product Algorithm 3 consumes).
    """
    r_n, hq, d = q.shape
    scale = d ** -0.5 if scale is None else scale
    out = torch.empty(r_n, hq, d, dtype=torch.float32, device=q.device)
    lse = torch.empty(r_n, hq, dtype=torch.float32, device=q.device)
    for r in range(r_n):
        k, v = gather_kv(kv, block_table, int(seq_used[r]), r)
        logits = _group_logits(q[r], k, scale)                        # [Hkv, G, S]
        lse[r] = torch.logsumexp(logits, -1).reshape(hq)
        probs = torch.softmax(logits, -1)
        out[r] = torch.matmul(probs, v.float().transpose(0, 1)).reshape(hq, d)
    return out, lse


def action_scores_ref(q, kv, block_table, seq_used, lse, out, n_seen, scale=None):
    """One action-query fold per request in torch (Algorithm 3): p = max over the GQA group of
    exp(scale * q . k - lse), folded into the running mean out += (p - out) / (n_seen + 1),
    then n_seen += 1.  Reference: lse_attn.py:63-78."""
    r_n, hq, d = q.shape
    scale = d ** -0.5 if scale is None else scale
    for r in range(r_n):
        s = int(seq_used[r])
        k, _ = gather_kv(kv, block_table, s, r)
        logits = _group_logits(q[r], k, scale)                        # [Hkv, G, S]
        p = torch.exp(logits - lse[r].reshape(logits.shape[0], -1, 1)).amax(1)
        cur = out[r, :, :s]
        cur += (p - cur) / (float(n_seen[r]) + 1.0)
    n_seen += 1
    return out


# ----------------------------------------------------------------------------- HIP path

def _as_i32(t: torch.Tensor, device) -> torch.Tensor:
    if t.dtype is not torch.int32 or t.get_device() != device.index:
        t = t.to(device=device, dtype=torch.int32)
    return t


def action_scores(q, kv, block_table, seq_used, lse, out, n_seen, scale=None, *,
                  n_valid=None, kv_len=None):
    """Fold the action query tokens of every request into `out` (Algorithm 3). In-place;
    returns `out`.

    q [R, Hq, D] (or [R, N, Hq, D], or [L, R, N, Hq, D]), kv [2, NB, BS, Hkv, D] (or
    [L, 2, NB, BS, Hkv, D]), block_table [R, MB] int32, seq_used [R] int32, lse [R, Hq]
    (or [R, N, Hq], [L, R, N, Hq]) fp32, out [R, Hkv, MB*BS] (or [L, R, Hkv, W]) fp32,
    n_seen [R] int32 (incremented by the number of folded queries).

    Reference: actkv/kernels/lse_attn.py:133-163.
    """
    span = block_table.shape[1] * kv.shape[-3]
    if out.shape[-1] < span:   # the kernel would write past each row
        raise ValueError(f"out is {out.shape[-1]} wide but the block table spans {span} slots; "
                         "allocate it as [R, Hkv, max_blocks * block_size]")
    dev = _hip.require_gpu("action_scores", q, kv, block_table, seq_used, lse, out, n_seen,
                           n_valid, kv_len)
    # strides are read as tuples and the K plane is addressed through the cache's own
    # pointer and strides (plane 0 starts at the cache's first element): each view or
    # per-dimension query would cost host time on every call
    kvs = kv.stride()
    multi_layer = kv.dim() == 6
    if multi_layer:
        L, _, nb, bs, hkv, d = kv.shape
        if q.dim() != 5 or lse.dim() != 4 or out.dim() != 4:
            raise ValueError("a [L, 2, NB, BS, Hkv, D] cache takes q [L, R, N, Hq, D], "
                             "lse [L, R, N, Hq] and out [L, R, Hkv, W]")
        q5, lse4, out4 = q, lse, out
        qs, ls, os_ = q.stride(), lse.stride(), out.stride()
        kv_sl = kvs[0]
    else:
        _, nb, bs, hkv, d = kv.shape
        L = 1
        if q.dim() == 3:        # one action token per request: the reference signature
            q5, lse4 = q.unsqueeze(1).unsqueeze(0), lse.unsqueeze(1).unsqueeze(0)
        elif q.dim() == 4:      # N action tokens per request
            q5, lse4 = q.unsqueeze(0), lse.unsqueeze(0)
        else:
            raise ValueError(f"q must be [R, Hq, D] or [R, N, Hq, D] for a one-layer cache, got {tuple(q.shape)}")
        out4 = out.unsqueeze(0)
        qs, ls, os_ = q5.stride(), lse4.stride(), out4.stride()
        kv_sl = 0
    _, r_n, n_q, hq, dq = q5.shape
    assert hq % hkv == 0
    assert dq == d
    assert kvs[-1] == 1 and qs[-1] == 1
    if lse4.dtype is not torch.float32 or out4.dtype is not torch.float32:
        raise TypeError("lse and out must be float32")
    if ls[-1] != 1 or os_[-1] != 1:
        raise ValueError("lse and out need a unit stride in their last dimension")
    if n_seen.dtype is not torch.int32:
        raise TypeError("n_seen must be int32 (it is updated in place)")
    if tuple(lse4.shape) != (L, r_n, n_q, hq) or tuple(out4.shape[:3]) != (L, r_n, hkv):
        raise ValueError(f"shape mismatch: q {tuple(q.shape)}, lse {tuple(lse.shape)}, out {tuple(out.shape)}")
    scale = scale if scale is not None else d ** -0.5
    bt = _as_i32(block_table, dev)
    if bt.stride(-1) != 1:
        bt = bt.contiguous()
    seq = _as_i32(seq_used, dev).contiguous()
    nv = None if n_valid is None else _as_i32(n_valid, dev).contiguous()
    kl = None if kv_len is None else _as_i32(kv_len, dev).contiguous()
    if kl is not None and tuple(kl.shape) != (r_n, n_q):
        raise ValueError(f"kv_len must be [R, N] = {(r_n, n_q)}")
    rc = _hip.glue().action_scores(
        q5.data_ptr(), _hip.dtype_code(q5.dtype), qs[0], qs[1], qs[2], qs[3],
        kv.data_ptr(), _hip.dtype_code(kv.dtype), kv_sl, kvs[-4], kvs[-3], kvs[-2],
        nb,
        bt.data_ptr(), bt.stride(0), bt.shape[1],
        seq.data_ptr(),
        lse4.data_ptr(), ls[0], ls[1], ls[2],
        out4.data_ptr(), os_[0], os_[1], os_[2], out4.shape[-1],
        n_seen.data_ptr(), _hip.ptr(nv), _hip.ptr(kl),
        L, r_n, n_q, hq, hkv, d, bs, float(scale), _hip.stream(dev))
    _hip.check(rc, "actkv_action_scores")
    return out


def paged_decode_attention(q, kv, block_table, seq_used, scale=None, *, n_valid=None, kv_len=None):
    """Paged attention with the LSE by-product on the GPU: returns (out, lse), float32.

    Same call and results as paged_decode_attention_ref (lse_attn.py:42-60), which stands in for
    the paged FlashAttention backend whose LSE Algorithm 3 consumes: q [R, Hq, D] ->
    out [R, Hq, D], lse [R, Hq].  Additive forms: q [R, N, Hq, D] (N queries per request) ->
    out [R, N, Hq, D], lse [R, N, Hq]; with kv [L, 2, NB, BS, Hkv, D], q [L, R, N, Hq, D] ->
    out [L, R, N, Hq, D], lse [L, R, N, Hq].  n_valid [R]: queries used per request (rows past it
    are zero); kv_len [R, N]: query n sees tokens t < kv_len[r, n] (causal limits).  A query
    that sees no token gets lse = -inf and out = 0.
    """
    dev = _hip.require_gpu("paged_decode_attention", q, kv, block_table, seq_used, n_valid, kv_len)
    if kv.dim() == 6:
        L, _, nb, bs, hkv, d = kv.shape
        if q.dim() != 5:
            raise ValueError("a [L, 2, NB, BS, Hkv, D] cache takes q [L, R, N, Hq, D]")
        q5, kv_sl, kv_sv, kv_k = q, kv.stride(0), kv.stride(1), kv[:, 0]
        squeeze = ()
    elif kv.dim() == 5:
        _, nb, bs, hkv, d = kv.shape
        L = 1
        if q.dim() == 3:
            q5, squeeze = q.unsqueeze(1).unsqueeze(0), (0, 2)
        elif q.dim() == 4:
            q5, squeeze = q.unsqueeze(0), (0,)
        else:
            raise ValueError(f"q must be [R, Hq, D] or [R, N, Hq, D] for a one-layer cache, got {tuple(q.shape)}")
        kv_sl, kv_sv, kv_k = 0, kv.stride(0), kv[0]
    else:
        raise ValueError(f"kv must be [2, NB, BS, Hkv, D] or [L, 2, NB, BS, Hkv, D], got {tuple(kv.shape)}")
    _, r_n, n_q, hq, dq = q5.shape
    assert hq % hkv == 0
    assert dq == d
    assert kv.stride(-1) == 1 and q.stride(-1) == 1
    scale = scale if scale is not None else d ** -0.5
    bt = _as_i32(block_table, dev)
    if bt.stride(-1) != 1:
        bt = bt.contiguous()
    seq = _as_i32(seq_used, dev).contiguous()
    nv = None if n_valid is None else _as_i32(n_valid, dev).contiguous()
    kl = None if kv_len is None else _as_i32(kv_len, dev).contiguous()
    if kl is not None and tuple(kl.shape) != (r_n, n_q):
        raise ValueError(f"kv_len must be [R, N] = {(r_n, n_q)}")
    alloc = torch.empty if nv is None else torch.zeros
    out = alloc(L, r_n, n_q, hq, d, dtype=torch.float32, device=dev)
    lse = alloc(L, r_n, n_q, hq, dtype=torch.float32, device=dev)
    lib = _hip.lib()
    nbytes = int(lib.actkv_paged_attention_workspace_size(L, r_n, n_q, hq, hkv, d, bt.shape[1], bs))
    ws = _hip.scratch(dev, "attention", nbytes) if nbytes else None
    rc = lib.actkv_paged_attention(
        q5.data_ptr(), _hip.dtype_code(q5.dtype), q5.stride(0), q5.stride(1), q5.stride(2), q5.stride(3),
        kv_k.data_ptr(), _hip.dtype_code(kv.dtype), kv_sl, kv_sv, kv_k.stride(-4), kv_k.stride(-3),
        kv_k.stride(-2), nb,
        bt.data_ptr(), bt.stride(0), bt.shape[1],
        seq.data_ptr(), _hip.ptr(nv), _hip.ptr(kl),
        out.data_ptr(), out.stride(0), out.stride(1), out.stride(2), out.stride(3),
        lse.data_ptr(), lse.stride(0), lse.stride(1), lse.stride(2),
        L, r_n, n_q, hq, hkv, d, bs, float(scale), _hip.ptr(ws), 0 if ws is None else ws.numel(),
        _hip.stream(dev))
    _hip.check(rc, "actkv_paged_attention")
    for dim in reversed(squeeze):
        out, lse = out.squeeze(dim), lse.squeeze(dim)
    return out, lse
