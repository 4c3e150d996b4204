"""Paged attention with the LSE by-product (actkv_paged_attention through
actkv.kernels.lse_attn.paged_decode_attention and PagedKVCache.decode_attention) against the
oracle's float64 restatement of lse_attn.py:42-60.

Tolerances:
- lse: absolute 1e-4. The logits are float32 MFMA dot products; the oracle is float64.
- out, matrix-core path: the probabilities enter the P.V product as two cache-dtype terms,
  hi = P rounded and lo = (P - hi) rounded, a relative error of about 2^-17 (bf16) or 2^-22
  (fp16) per term; with the float32 logits and exp, out is within ~1e-5 of the float64 oracle
  for |v| of a few units: atol 2e-4 for both dtypes (the reference's own outputs_match
  criterion is 1e-3, bench_kernels.py:129-131).
- out, float32 path: 1e-4.
"""
import math

import numpy as np
import pytest
import torch

from actkv.kernels.lse_attn import paged_decode_attention
from actkv.paged import PagedKVCache
from oracle import reference as ref

pytestmark = pytest.mark.gpu


def _cache(lens, layers=1, hkv=8, d=128, bs=16, dtype=torch.bfloat16, seed=0):
    g = torch.Generator().manual_seed(seed)
    nb = sum(math.ceil(n / bs) for n in lens) + 5
    cache = PagedKVCache(nb, bs, hkv, d, n_layers=layers, dtype=dtype, device="cuda")
    cache.free = torch.randperm(nb, generator=g).tolist()
    for r, n in enumerate(lens):
        k = torch.randn(layers, n, hkv, d, generator=g).to(dtype)
        v = torch.randn(layers, n, hkv, d, generator=g).to(dtype)
        cache.append(r, k.cuda(), v.cuda())
    return cache


def _oracle(cache, reqs, q, layer, kv_len=None, n_valid=None):
    """q [R, N, Hq, D] (CPU) -> oracle (out, lse) for one layer."""
    kvl = cache.kv[layer].cpu()
    tables = [cache.tables[r] for r in reqs]
    seqs = [cache.seq_used[r] for r in reqs]
    return ref.paged_attention(q.float(), kvl.float(), tables, seqs, kv_len=kv_len, n_valid=n_valid)


def _atol(dtype):
    return {torch.bfloat16: 2e-4, torch.float16: 2e-4, torch.float32: 1e-4}[dtype]


@pytest.mark.parametrize("lens,hq,hkv,n_q,dtype,causal", [
    ([700, 1500], 32, 8, 1, torch.bfloat16, False),      # decode: one 32-row tile, 4 real rows
    ([2000, 1337], 32, 8, 64, torch.bfloat16, True),     # action region: 256 rows, causal limits
    ([900], 16, 8, 40, torch.float16, False),            # GQA 2, 80 rows (3 tiles)
    ([1100, 64], 8, 8, 100, torch.bfloat16, True),       # GQA 1, 100 rows, a short request
    ([640], 32, 8, 200, torch.bfloat16, True),           # 800 rows: four groups of 8 tiles
    ([3000, 47], 32, 8, 8, torch.bfloat16, True),        # 32 rows: the one-tile decode kernel, causal
    ([2100], 16, 8, 5, torch.float16, True),             # GQA 2, 10 rows, fp16, causal
    ([5000, 1], 8, 8, 3, torch.bfloat16, False),         # GQA 1, 3 rows, a one-token request
    ([1800, 333], 64, 8, 48, torch.bfloat16, True),      # GQA 8, 384 rows, causal
    ([2500], 16, 2, 100, torch.float16, False),          # GQA 8, 800 rows: four groups of 8 tiles
    ([700, 4100], 64, 8, 1, torch.bfloat16, False),      # GQA 8 decode: one tile, 8 real rows
    ([3000, 47], 64, 8, 4, torch.bfloat16, True),        # GQA 8, 32 rows: the one-tile decode kernel
    ([1800, 333], 24, 8, 30, torch.bfloat16, True),      # GQA 3, 90 rows
    ([2500], 40, 8, 20, torch.float16, False),           # GQA 5, 100 rows
    ([700], 48, 8, 60, torch.bfloat16, True),            # GQA 6, 360 rows
    ([1200, 900], 28, 4, 5, torch.bfloat16, True),       # GQA 7, 35 rows (two tiles)
    ([3000, 47], 28, 4, 4, torch.float16, True),         # GQA 7, 28 rows: the decode kernel
])
def test_matrix_core_path_matches_the_oracle(lens, hq, hkv, n_q, dtype, causal):
    cache = _cache(lens, hkv=hkv, dtype=dtype, seed=len(lens) * 100 + n_q)
    reqs = list(range(len(lens)))
    g = torch.Generator().manual_seed(n_q)
    q = torch.randn(len(lens), n_q, hq, 128, generator=g).to(dtype)
    kv_len = None
    if causal:
        kv_len = torch.stack([torch.randint(0, S + 8, (n_q,), generator=g) for S in lens]).to(torch.int32)
        kv_len[0, 0] = 0                                           # a query that sees nothing
    out, lse = cache.decode_attention(reqs, q.cuda(), kv_len=None if kv_len is None else kv_len.cuda())
    want_out, want_lse = _oracle(cache, reqs, q, 0, kv_len=None if kv_len is None else kv_len.tolist())
    torch.testing.assert_close(lse.cpu(), want_lse, rtol=0, atol=1e-4)
    torch.testing.assert_close(out.cpu(), want_out, rtol=0, atol=_atol(dtype))
    if causal:
        assert float(lse[0, 0, 0]) == -math.inf and torch.equal(out[0, 0].cpu(), torch.zeros(hq, 128))


@pytest.mark.parametrize("lens,hq,hkv,n_q,dtype,causal,bs,split", [
    ([700, 1500], 32, 8, 1, torch.bfloat16, False, 16, True),    # decode: 4 real rows
    ([3000, 47], 64, 8, 4, torch.bfloat16, True, 16, True),      # GQA 8 decode tile, causal
    ([3000, 47], 64, 8, 4, torch.float16, True, 16, False),      # the same in one pass, fp16
    ([900], 16, 8, 20, torch.float16, False, 16, True),          # GQA 2, 40 rows: 2-wave ring
    ([2000, 1337], 32, 8, 30, torch.bfloat16, True, 16, True),   # 120 rows: 4-wave ring
    ([640], 32, 8, 200, torch.bfloat16, True, 16, True),         # 800 rows: 8-wave ring groups
    ([640, 2200], 32, 8, 200, torch.bfloat16, True, 16, False),  # the same in one pass
    ([2500], 64, 8, 50, torch.float16, False, 32, True),         # GQA 8, 400 rows, block 32
    ([5000, 700], 8, 2, 48, torch.bfloat16, True, 256, True),    # chunk starts inside blocks
    ([4400, 1], 56, 8, 1, torch.bfloat16, False, 64, True),      # GQA 7 decode, a one-token request
    ([1800, 333], 24, 8, 30, torch.bfloat16, True, 16, True),    # GQA 3, 90 rows
    ([1500, 300], 32, 2, 3, torch.bfloat16, True, 16, True),     # GQA 16, 48 rows: 2-wave ring
    ([2000, 900], 64, 2, 1, torch.float16, False, 32, True),     # GQA 32 decode: one full tile
])
def test_matrix_core_path_head_dim_64(monkeypatch, lens, hq, hkv, n_q, dtype, causal, bs, split):
    """Head dim 64 on the matrix-core kernels (128-byte token rows: eight rows per 16-byte
    load instruction, their own LDS swizzle, two 32-dim output tiles), every kernel form,
    with and without the token split, against the oracle at the same tolerances."""
    from actkv import _hip
    cache = _cache(lens, hkv=hkv, d=64, bs=bs, dtype=dtype, seed=len(lens) * 100 + n_q + bs)
    reqs = list(range(len(lens)))
    g = torch.Generator().manual_seed(n_q + 64)
    q = torch.randn(len(lens), n_q, hq, 64, generator=g).to(dtype)
    kv_len = None
    if causal:
        kv_len = torch.stack([torch.randint(0, S + 8, (n_q,), generator=g) for S in lens]).to(torch.int32)
        kv_len[0, 0] = 0                                           # a query that sees nothing
    lib = _hip.lib()
    mb = max(len(t) for t in cache.tables.values())
    if split:
        assert lib.actkv_paged_attention_workspace_size(1, len(lens), n_q, hq, hkv, 64, mb, bs) > 0
    else:
        monkeypatch.setattr(lib, "actkv_paged_attention_workspace_size", lambda *a: 0)
    out, lse = cache.decode_attention(reqs, q.cuda(), kv_len=None if kv_len is None else kv_len.cuda())
    want_out, want_lse = _oracle(cache, reqs, q, 0, kv_len=None if kv_len is None else kv_len.tolist())
    torch.testing.assert_close(lse.cpu(), want_lse, rtol=0, atol=1e-4)
    torch.testing.assert_close(out.cpu(), want_out, rtol=0, atol=_atol(dtype))
    if causal:
        assert float(lse[0, 0, 0]) == -math.inf and torch.equal(out[0, 0].cpu(), torch.zeros(hq, 64))


def test_reference_signature_one_query_per_request():
    """q [R, Hq, D] -> out [R, Hq, D], lse [R, Hq], as paged_decode_attention_ref."""
    cache = _cache([333, 1024, 17], seed=5)
    q = torch.randn(3, 32, 128, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    out, lse = cache.decode_attention([0, 1, 2], q.cuda())
    assert tuple(out.shape) == (3, 32, 128) and tuple(lse.shape) == (3, 32)
    want_out, want_lse = _oracle(cache, [0, 1, 2], q.unsqueeze(1), 0)
    torch.testing.assert_close(lse.cpu(), want_lse[:, 0], rtol=0, atol=1e-4)
    torch.testing.assert_close(out.cpu(), want_out[:, 0], rtol=0, atol=_atol(cache.kv.dtype))


def test_all_layers_with_ragged_query_counts():
    """layer=None: q [L, R, N, Hq, D]; n_valid leaves the unused rows at zero."""
    layers = 3
    cache = _cache([500, 260], layers=layers, seed=7)
    g = torch.Generator().manual_seed(8)
    n_q = 24
    q = torch.randn(layers, 2, n_q, 32, 128, generator=g).to(torch.bfloat16)
    n_valid = torch.tensor([24, 9], dtype=torch.int32)
    out, lse = cache.decode_attention([0, 1], q.cuda(), layer=None, n_valid=n_valid.cuda())
    assert tuple(out.shape) == (layers, 2, n_q, 32, 128)
    for l in range(layers):
        want_out, want_lse = _oracle(cache, [0, 1], q[l], l, n_valid=n_valid.tolist())
        torch.testing.assert_close(lse[l].cpu(), want_lse, rtol=0, atol=1e-4)
        torch.testing.assert_close(out[l].cpu(), want_out, rtol=0, atol=_atol(cache.kv.dtype))
    assert torch.equal(out[:, 1, 9:].cpu(), torch.zeros(layers, n_q - 9, 32, 128))


@pytest.mark.parametrize("n0,n_q", [(40, 2), (3000, 2), (3000, 40)])
def test_empty_sequence_gives_minus_inf_and_zero(n0, n_q):
    """An empty request next to another: one pass, the decode kernel's split, the ring
    kernel's split (its combine merges no chunk for the empty request)."""
    cache = _cache([n0, 0], seed=9)
    assert cache.seq_used[1] == 0
    q = torch.randn(2, n_q, 32, 128).to(torch.bfloat16)
    out, lse = cache.decode_attention([0, 1], q.cuda())
    assert torch.isinf(lse[1]).all() and (lse[1] < 0).all()
    assert torch.equal(out[1].cpu(), torch.zeros(n_q, 32, 128))
    want_out, want_lse = _oracle(cache, [0], q[:1], 0)
    torch.testing.assert_close(lse[:1].cpu(), want_lse, rtol=0, atol=1e-4)


@pytest.mark.parametrize("d,hq,hkv,bs,dtype", [
    (96, 8, 2, 16, torch.bfloat16),      # head_dim 96
    (32, 4, 2, 16, torch.float32),       # float32 cache
    (128, 12, 4, 12, torch.float16),     # GQA 3, block size 12
])
def test_float32_path_matches_the_oracle(d, hq, hkv, bs, dtype):
    cache = _cache([150, 77], hkv=hkv, d=d, bs=bs, dtype=dtype, seed=d + hq)
    g = torch.Generator().manual_seed(bs)
    q = torch.randn(2, 5, hq, d, generator=g).to(dtype)
    kv_len = torch.tensor([[150, 3, 0, 90, 151], [1, 77, 40, 2, 60]], dtype=torch.int32)
    out, lse = cache.decode_attention([0, 1], q.cuda(), kv_len=kv_len.cuda())
    want_out, want_lse = _oracle(cache, [0, 1], q, 0, kv_len=kv_len.tolist())
    torch.testing.assert_close(lse.cpu(), want_lse, rtol=0, atol=1e-4)
    torch.testing.assert_close(out.cpu(), want_out, rtol=0, atol=1e-4)


@pytest.mark.parametrize("lens,n_q,hq,hkv,d,bs,dtype,causal,split", [
    ([4000, 2500], 1, 16, 8, 256, 16, torch.bfloat16, False, True),   # head dim 256 decode (Gemma shape), split
    ([4000, 2500], 1, 16, 8, 256, 16, torch.bfloat16, False, False),  # the same in one pass
    ([3000, 47], 3, 8, 2, 30, 12, torch.float16, True, True),         # head dim 30, block 12, causal
    ([900], 9, 8, 2, 96, 16, torch.bfloat16, True, True),             # 36 rows: three row groups
    ([2100, 0, 5], 1, 40, 1, 80, 8, torch.float32, False, True),      # G 40, an empty request, fp32
    ([1300], 20, 32, 8, 128, 16, torch.float32, True, False),         # fp32 cache, 80 rows, one pass
])
def test_float32_path_row_groups_and_token_split(monkeypatch, lens, n_q, hq, hkv, d, bs, dtype, causal, split):
    """The float32 path takes up to 16 query rows of one KV head per workgroup over a token
    chunk (the chunks merged by the combine launch when a workspace is given): head dims off
    the matrix cores, blocks that are not a power of two, GQA groups wider than a row group,
    empty requests, causal limits, with and without the split, against the oracle."""
    from actkv import _hip
    cache = _cache(lens, hkv=hkv, d=d, bs=bs, dtype=dtype, seed=d + n_q + bs)
    reqs = list(range(len(lens)))
    g = torch.Generator().manual_seed(d + hq)
    q = torch.randn(len(lens), n_q, hq, d, generator=g).to(dtype)
    kv_len = None
    if causal:
        kv_len = torch.stack([torch.randint(0, S + 8, (n_q,), generator=g) for S in lens]).to(torch.int32)
        kv_len[0, 0] = 0
    lib = _hip.lib()
    mb = max(len(t) for t in cache.tables.values())
    if split:
        assert lib.actkv_paged_attention_workspace_size(1, len(lens), n_q, hq, hkv, d, mb, bs) > 0
    else:
        monkeypatch.setattr(lib, "actkv_paged_attention_workspace_size", lambda *a: 0)
    out, lse = cache.decode_attention(reqs, q.cuda(), kv_len=None if kv_len is None else kv_len.cuda())
    want_out, want_lse = _oracle(cache, reqs, q, 0, kv_len=None if kv_len is None else kv_len.tolist())
    torch.testing.assert_close(lse.cpu(), want_lse, rtol=0, atol=1e-4)
    torch.testing.assert_close(out.cpu(), want_out, rtol=0, atol=1e-4)


def test_device_lse_drives_action_scoring():
    """Algorithm 3 end to end on the device: the attention kernel's lse, fed to cal_attn, gives
    the oracle's scores computed with the oracle's lse (within the scoring tolerance)."""
    cache = _cache([1200, 800], seed=11)
    g = torch.Generator().manual_seed(12)
    n_q = 32
    q = torch.randn(2, n_q, 32, 128, generator=g).to(torch.bfloat16)
    S = [1200, 800]
    kv_len = torch.stack([torch.arange(s - n_q + 1, s + 1) for s in S]).to(torch.int32)
    _, lse = cache.decode_attention([0, 1], q.cuda(), kv_len=kv_len.cuda())
    width = max(len(cache.tables[r]) for r in (0, 1)) * 16
    out = torch.zeros(2, 8, width, device="cuda")
    n_seen = torch.zeros(2, dtype=torch.int32, device="cuda")
    cache.cal_attn([0, 1], q.cuda(), lse, out, n_seen, layer=0, kv_len=kv_len.cuda())
    _, lse_o = _oracle(cache, [0, 1], q, 0, kv_len=kv_len.tolist())
    want = torch.zeros(2, 8, width)
    kvl = cache.kv[0].cpu()
    for r in range(2):
        s = cache.seq_used[r]
        k = ref.gather_k(kvl, cache.tables[r], s).double().repeat_interleave(4, dim=1)
        for n in range(n_q):
            lim = int(kv_len[r, n])
            logits = torch.einsum("hd,shd->hs", q[r, n].double(), k[:lim]) * 128 ** -0.5
            p = torch.exp(logits - lse_o[r, n].double().unsqueeze(-1)).view(8, 4, lim).amax(1)
            want[r, :, :lim] += p.float() / n_q
    torch.testing.assert_close(out.cpu(), want, rtol=1e-3, atol=1e-6)


@pytest.mark.parametrize("n_q", [16, 8, 1])
def test_token_split_and_single_pass_agree(monkeypatch, n_q):
    """With a workspace, long sequences are split into token chunks and merged by the combine
    launch; without one, one workgroup attends the whole sequence. Both match the oracle.
    16 queries take the multi-tile kernel, 8 and 1 the one-tile decode kernel."""
    from actkv import _hip
    cache = _cache([4000, 2500], seed=13)
    g = torch.Generator().manual_seed(14)
    q = torch.randn(2, n_q, 32, 128, generator=g).to(torch.bfloat16)
    kv_len = torch.stack([torch.randint(1, S + 1, (n_q,), generator=g) for S in (4000, 2500)]).to(torch.int32)
    lib = _hip.lib()
    assert lib.actkv_paged_attention_workspace_size(1, 2, n_q, 32, 8, 128, len(cache.tables[0]), 16) > 0
    split_out, split_lse = cache.decode_attention([0, 1], q.cuda(), kv_len=kv_len.cuda())
    monkeypatch.setattr(lib, "actkv_paged_attention_workspace_size", lambda *a: 0)
    one_out, one_lse = cache.decode_attention([0, 1], q.cuda(), kv_len=kv_len.cuda())
    want_out, want_lse = _oracle(cache, [0, 1], q, 0, kv_len=kv_len.tolist())
    for out, lse in ((split_out, split_lse), (one_out, one_lse)):
        torch.testing.assert_close(lse.cpu(), want_lse, rtol=0, atol=1e-4)
        torch.testing.assert_close(out.cpu(), want_out, rtol=0, atol=_atol(cache.kv.dtype))


@pytest.mark.parametrize("bs,lens,n_q,causal,split", [
    (32, [3000, 1111], 40, True, True),      # ring kernel (160 rows), block 32
    (64, [2600], 8, False, True),            # decode kernel (32 rows), block 64
    (256, [5000, 700], 48, True, True),      # ring kernel; chunk starts are not block-aligned
    (256, [5000], 3, True, False),           # decode kernel, one pass
    (128, [3333], 100, False, False),        # ring kernel, one pass, 400 rows in two groups
])
def test_block_sizes_and_chunking(monkeypatch, bs, lens, n_q, causal, split):
    """The matrix-core kernels take any power-of-two block of at least 16 tokens: the ring
    kernel's loads are per block and its block-table window is indexed by block."""
    from actkv import _hip
    cache = _cache(lens, hkv=2, bs=bs, seed=bs + n_q)
    reqs = list(range(len(lens)))
    g = torch.Generator().manual_seed(bs)
    q = torch.randn(len(lens), n_q, 8, 128, generator=g).to(torch.bfloat16)
    kv_len = None
    if causal:
        kv_len = torch.stack([torch.randint(1, S + 1, (n_q,), generator=g) for S in lens]).to(torch.int32)
    lib = _hip.lib()
    if split:
        assert lib.actkv_paged_attention_workspace_size(1, len(lens), n_q, 8, 2, 128,
                                                        max(len(t) for t in cache.tables.values()), bs) > 0
    else:
        monkeypatch.setattr(lib, "actkv_paged_attention_workspace_size", lambda *a: 0)
    out, lse = cache.decode_attention(reqs, q.cuda(), kv_len=None if kv_len is None else kv_len.cuda())
    want_out, want_lse = _oracle(cache, reqs, q, 0, kv_len=None if kv_len is None else kv_len.tolist())
    torch.testing.assert_close(lse.cpu(), want_lse, rtol=0, atol=1e-4)
    torch.testing.assert_close(out.cpu(), want_out, rtol=0, atol=_atol(cache.kv.dtype))


def test_block_table_window_refill(monkeypatch):
    """One workgroup attends 70k tokens of 16-token blocks in one pass: more blocks than the
    ring kernel's LDS table window holds (4096), so the window is refilled mid-sequence."""
    from actkv import _hip
    cache = _cache([70000], hkv=1, seed=21)
    g = torch.Generator().manual_seed(22)
    q = torch.randn(1, 40, 4, 128, generator=g).to(torch.bfloat16)     # 160 rows: 8-wave groups
    monkeypatch.setattr(_hip.lib(), "actkv_paged_attention_workspace_size", lambda *a: 0)
    out, lse = cache.decode_attention([0], q.cuda())
    want_out, want_lse = _oracle(cache, [0], q, 0)
    torch.testing.assert_close(lse.cpu(), want_lse, rtol=0, atol=1e-4)
    torch.testing.assert_close(out.cpu(), want_out, rtol=0, atol=_atol(cache.kv.dtype))


@pytest.mark.parametrize("lens,hq,hkv,widen,causal", [
    ([4400, 3000, 1, 4400], 32, 8, 2, False),        # table twice as wide as the sequences
    ([4400, 2900], 32, 8, 3, True),                  # the same, causal limits
    ([20000], 4, 1, 1, False),                       # one pair: 125 chunks, merged 64 at a time
    ([50 + 7 * i for i in range(70)], 4, 1, 2, False),  # 70 requests: the longest is found across lanes
])
def test_decode_split_follows_the_longest_sequence(lens, hq, hkv, widen, causal):
    """The decode kernel's chunk length is the longest sequence of the call over the chunk
    count, whatever the block table's width (a wider table gives the same bits), and the
    combine merges any number of chunks."""
    from actkv import _hip
    bs = 16
    cache = _cache(lens, hkv=hkv, bs=bs, seed=len(lens) + hq)
    reqs = list(range(len(lens)))
    seq, bt = cache._device_tables(reqs)
    wide = torch.zeros(len(lens), bt.shape[1] * widen, dtype=torch.int32, device="cuda")
    wide[:, : bt.shape[1]] = bt
    assert _hip.lib().actkv_paged_attention_workspace_size(1, len(lens), 1, hq, hkv, 128, wide.shape[1], bs) > 0
    g = torch.Generator().manual_seed(len(lens))
    q = torch.randn(len(lens), 1, hq, 128, generator=g).to(torch.bfloat16)
    kv_len = None
    if causal:
        kv_len = torch.stack([torch.randint(1, S + 1, (1,), generator=g) for S in lens]).to(torch.int32)
    out, lse = paged_decode_attention(q.cuda(), cache.kv[0], wide, seq,
                                      kv_len=None if kv_len is None else kv_len.cuda())
    want_out, want_lse = _oracle(cache, reqs, q, 0, kv_len=None if kv_len is None else kv_len.tolist())
    torch.testing.assert_close(lse.cpu(), want_lse, rtol=0, atol=1e-4)
    torch.testing.assert_close(out.cpu(), want_out, rtol=0, atol=_atol(cache.kv.dtype))
    # the split does not depend on the table's width: the tight table gives the same bits
    tight_out, tight_lse = paged_decode_attention(q.cuda(), cache.kv[0], bt, seq,
                                                  kv_len=None if kv_len is None else kv_len.cuda())
    assert torch.equal(tight_out, out) and torch.equal(tight_lse, lse)


def test_split_calls_of_different_shapes_share_the_workspace():
    """Decode calls of different shapes, back to back on one workspace: each merges its own
    chunks, whatever an earlier call of another shape left in the workspace."""
    shapes = [([700, 1500], 32, 8), ([333, 1024, 17], 32, 8), ([4000], 4, 1), ([700, 1500], 32, 8)]
    for i, (lens, hq, hkv) in enumerate(shapes):
        cache = _cache(lens, hkv=hkv, seed=40 + i)
        reqs = list(range(len(lens)))
        q = torch.randn(len(lens), 1, hq, 128, generator=torch.Generator().manual_seed(i)).to(torch.bfloat16)
        out, lse = cache.decode_attention(reqs, q.cuda())
        want_out, want_lse = _oracle(cache, reqs, q, 0)
        torch.testing.assert_close(lse.cpu(), want_lse, rtol=0, atol=1e-4)
        torch.testing.assert_close(out.cpu(), want_out, rtol=0, atol=_atol(cache.kv.dtype))


def test_many_pairs_take_one_pass_without_a_workspace():
    """36 layers x 29 requests x 8 KV heads = 8352 pairs, 16 rounds of resident workgroups:
    the decode kernel attends each pair in one pass and asks for no workspace; the first and
    last layers match the oracle."""
    from actkv import _hip
    layers, lens = 36, [40 + 7 * i for i in range(29)]
    cache = _cache(lens, layers=layers, seed=31)
    reqs = list(range(len(lens)))
    width = max(len(cache.tables[r]) for r in reqs)
    assert _hip.lib().actkv_paged_attention_workspace_size(layers, len(lens), 1, 32, 8, 128, width, 16) == 0
    q = torch.randn(layers, len(lens), 1, 32, 128, generator=torch.Generator().manual_seed(32)).to(torch.bfloat16)
    out, lse = cache.decode_attention(reqs, q.cuda(), layer=None)
    for l in (0, layers - 1):
        want_out, want_lse = _oracle(cache, reqs, q[l], l)
        torch.testing.assert_close(lse[l].cpu(), want_lse, rtol=0, atol=1e-4)
        torch.testing.assert_close(out[l].cpu(), want_out, rtol=0, atol=_atol(cache.kv.dtype))
