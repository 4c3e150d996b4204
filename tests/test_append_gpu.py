"""Device append and slot map (actkv_append / actkv_slot_map) against the oracle's paged cache.

The cache bytes after a sequence of appends must equal, bit for bit, the oracle model's after
the same appends of the sources converted by torch on the CPU (the reference's own `.to()`):
every cache dtype x source dtype, ragged chunks that cross block boundaries, a shuffled free
stack, broadcast and strided sources, head dims that take the one-element-per-thread kernel,
and batched appends over several requests.  Allocator state (tables, free stack, seq_used)
must match exactly.  Reference: actkv/paged.py:67-97."""
import numpy as np
import pytest
import torch

from actkv import _hip
from actkv.paged import OutOfBlocks, PagedKVCache
from oracle import reference as ref

pytestmark = pytest.mark.gpu

_NP = {torch.float32: np.float32, torch.float16: np.uint16, torch.bfloat16: np.uint16}


def _bits_np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float32:
        return t.numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


def _source(shape, dtype, g):
    """Values that exercise rounding: normal draws over several magnitudes, bf16 halfway
    points (low 16 bits 0x8000), values that overflow fp16, fp16 subnormals."""
    x = torch.randn(*shape, generator=g) * torch.tensor([1.0, 1e-3, 300.0, 7e4])[
        torch.randint(0, 4, shape, generator=g)]
    flat = x.view(-1)
    n = flat.numel()
    half = (flat[: n // 8].view(torch.int32) & ~0xFFFF) | 0x8000
    flat[: n // 8] = half.view(torch.float32)
    flat[n // 8: n // 8 + 16] = torch.tensor([1e5, -1e5, 6.1e-5, 3e-8, -2e-7, 65504.0, 65520.0, -65519.0,
                                              0.0, -0.0, 1.0, -1.0, 2.0 ** -24, 2.0 ** -25, 3.0 * 2.0 ** -26,
                                              1e-40])[: min(16, n - n // 8)]
    return x.to(dtype)


def _pair(nb, bs, hkv, d, layers, kv_dtype, seed):
    g = torch.Generator().manual_seed(seed)
    cache = PagedKVCache(nb, bs, hkv, d, n_layers=layers, dtype=kv_dtype, device="cuda")
    model = ref.PagedCacheModel(nb, bs, hkv, d, layers, np_dtype=_NP[kv_dtype])
    order = torch.randperm(nb, generator=g).tolist()
    cache.free = list(order)
    model.free = list(order)
    return cache, model, g


def _same(cache, model):
    torch.cuda.synchronize()
    got = _bits_np(cache.kv)
    assert got.shape == model.kv.shape
    diff = np.nonzero(got.view(np.uint8) != model.kv.view(np.uint8))[0]
    assert diff.size == 0, f"{diff.size} bytes differ, first at byte {diff[:4]}"
    assert cache.free == model.free
    assert {r: list(t) for r, t in cache.tables.items()} == model.tables
    assert cache.seq_used == model.seq_used


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("src_dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_append_matches_the_oracle_model(kv_dtype, src_dtype):
    layers, hkv, d, bs = 3, 8, 128, 16
    cache, model, g = _pair(64, bs, hkv, d, layers, kv_dtype, seed=11)
    for req, n in [(0, 5), (1, 16), (0, 1), (0, 37), (2, 0), (1, 250), (0, 10)]:
        k = _source((layers, n, hkv, d), src_dtype, g)
        v = _source((layers, n, hkv, d), src_dtype, g)
        cache.append(req, k.cuda(), v.cuda())
        model.append(req, _bits_np(k.to(kv_dtype)), _bits_np(v.to(kv_dtype)))
    _same(cache, model)


@pytest.mark.parametrize("d", [12, 4, 40])
def test_unaligned_head_dims_and_strided_sources(d):
    """D not a multiple of 8 (one element per thread) and sources whose rows are views into
    a wider tensor, so no row starts 16-byte aligned."""
    layers, hkv, bs = 2, 3, 8
    cache, model, g = _pair(40, bs, hkv, d, layers, torch.bfloat16, seed=5)
    for req, n in [(0, 3), (0, 9), (1, 17), (0, 40)]:
        wide_k = _source((layers, n, hkv, d + 3), torch.float32, g)
        wide_v = _source((layers, n, hkv, d + 1), torch.float32, g)
        k, v = wide_k[..., 1: d + 1], wide_v[..., :d]
        cache.append(req, k.cuda(), v.cuda())
        model.append(req, _bits_np(k.to(torch.bfloat16)), _bits_np(v.to(torch.bfloat16)))
    _same(cache, model)


def test_broadcast_cpu_and_mixed_sources():
    """A source with one layer broadcasts over the layers (as the reference's indexed
    assignment does), CPU sources are moved first, and k and v of different dtypes are each
    converted straight to the cache dtype; float64 takes torch's own conversion."""
    layers, hkv, d, bs = 4, 2, 64, 16
    cache, model, g = _pair(24, bs, hkv, d, layers, torch.float16, seed=9)
    k = _source((1, 21, hkv, d), torch.float32, g)
    v = _source((layers, 21, hkv, d), torch.float32, g)
    cache.append(0, k.cuda(), v)                                  # v stays on the CPU
    model.append(0, _bits_np(k.to(torch.float16).expand(layers, -1, -1, -1)), _bits_np(v.to(torch.float16)))
    k = _source((layers, 11, hkv, d), torch.float32, g)
    v = _source((layers, 11, hkv, d), torch.bfloat16, g)
    cache.append(0, k.cuda(), v.cuda())
    model.append(0, _bits_np(k.to(torch.float16)), _bits_np(v.to(torch.float16)))
    k = _source((layers, 7, hkv, d), torch.float32, g).double()
    v = _source((layers, 7, hkv, d), torch.float32, g).double()
    cache.append(0, k.cuda(), v.cuda())
    model.append(0, _bits_np(k.to(torch.float16)), _bits_np(v.to(torch.float16)))
    _same(cache, model)


def test_append_batch_equals_appends_in_order():
    layers, hkv, d, bs = 2, 8, 128, 16
    cache, model, g = _pair(96, bs, hkv, d, layers, torch.bfloat16, seed=3)
    # prefill three requests, then a decode step (one token each), then ragged chunks
    for req, n in [(0, 30), (1, 16), (2, 1)]:
        k = _source((layers, n, hkv, d), torch.bfloat16, g)
        v = _source((layers, n, hkv, d), torch.bfloat16, g)
        cache.append(req, k.cuda(), v.cuda())
        model.append(req, _bits_np(k), _bits_np(v))
    for reqs, counts in [([0, 1, 2], None), ([2, 0, 3, 1], [40, 0, 17, 1]), ([1, 3], [15, 16])]:
        cnt = [1] * len(reqs) if counts is None else counts
        k = _source((layers, sum(cnt), hkv, d), torch.float32, g)
        v = _source((layers, sum(cnt), hkv, d), torch.float32, g)
        cache.append_batch(reqs, k.cuda(), v.cuda(), counts)
        o = 0
        for r, c in zip(reqs, cnt):
            model.append(r, _bits_np(k[:, o: o + c].to(torch.bfloat16)), _bits_np(v[:, o: o + c].to(torch.bfloat16)))
            o += c
    _same(cache, model)
    with pytest.raises(ValueError):
        cache.append_batch([0, 0], torch.zeros(layers, 2, hkv, d, device="cuda"),
                           torch.zeros(layers, 2, hkv, d, device="cuda"))


def test_slot_map_and_gather_follow_evictions():
    layers, hkv, d, bs = 2, 2, 32, 4
    cache, model, g = _pair(30, bs, hkv, d, layers, torch.bfloat16, seed=21)
    k = _source((layers, 45, hkv, d), torch.bfloat16, g)
    v = _source((layers, 45, hkv, d), torch.bfloat16, g)
    cache.append(0, k.cuda(), v.cuda())
    model.append(0, _bits_np(k), _bits_np(v))
    for n in (None, 0, 1, 13, 44, 48):
        got = cache.slot_map(0, n)
        assert got.dtype == torch.int64 and got.is_cuda
        assert np.array_equal(got.cpu().numpy(), model.slot_map(0, n))
    with pytest.raises(IndexError):
        cache.slot_map(0, 49)
    keep = torch.zeros(45, dtype=torch.bool)
    keep[::3] = True
    perm = cache.compact(0, keep.cuda())
    perm_m = model.compact(0, keep.numpy())
    assert perm.cpu().numpy().tolist() == perm_m.tolist()
    assert np.array_equal(cache.slot_map(0).cpu().numpy(), model.slot_map(0))
    gk, gv = cache.gather(0, layer=1)
    mk, mv = model.gather(0, layer=1)
    assert np.array_equal(_bits_np(gk), mk) and np.array_equal(_bits_np(gv), mv)
    # appending after a compaction continues from the survivors' blocks
    k = _source((layers, 9, hkv, d), torch.bfloat16, g)
    cache.append(0, k.cuda(), k.cuda())
    model.append(0, _bits_np(k), _bits_np(k))
    _same(cache, model)


def test_out_of_blocks_leaves_the_cache_unchanged():
    cache = PagedKVCache(4, 16, 2, 64, n_layers=1, dtype=torch.bfloat16, device="cuda")
    before = cache.kv.clone()
    with pytest.raises(OutOfBlocks):
        cache.append(0, torch.ones(1, 65, 2, 64, device="cuda"), torch.ones(1, 65, 2, 64, device="cuda"))
    assert torch.equal(cache.kv, before) and cache.free == [3, 2, 1, 0]


def test_abi_flags_missing_blocks_and_writes_the_rest():
    """A token whose block is missing from the table (or outside the pool) is skipped and
    flagged; every other token is written."""
    L, nb, bs, hkv, d = 1, 4, 4, 1, 8
    kv = torch.zeros(L, 2, nb, bs, hkv, d, dtype=torch.float32, device="cuda")
    k = torch.arange(12 * d, dtype=torch.float32, device="cuda").view(1, 12, 1, d) + 1
    table = torch.tensor([[2, 9, -1]], dtype=torch.int32, device="cuda")   # block 1: outside, block 2: -1
    starts = torch.tensor([0], dtype=torch.int32, device="cuda")
    counts = torch.tensor([12], dtype=torch.int32, device="cuda")
    off = torch.tensor([0], dtype=torch.int64, device="cuda")
    bad = torch.zeros(1, dtype=torch.int32, device="cuda")
    s = kv.stride()
    rc = _hip.lib().actkv_append(kv.data_ptr(), _hip.dtype_code(kv.dtype), s[0], s[1], s[2], s[3], s[4], nb,
                                 k.data_ptr(), k.data_ptr(), _hip.dtype_code(k.dtype), *k.stride()[:3],
                                 *k.stride()[:3], L, hkv, d, 1, starts.data_ptr(), counts.data_ptr(),
                                 off.data_ptr(), 12, table.data_ptr(), 3, 3, bs, bad.data_ptr(),
                                 _hip.stream(kv.device))
    _hip.check(rc, "actkv_append")
    torch.cuda.synchronize()
    assert int(bad) == 1
    assert torch.equal(kv[0, 0, 2].view(4, d), k[0, :4, 0]) and torch.equal(kv[0, 1, 2].view(4, d), k[0, :4, 0])
    others = torch.ones(nb, dtype=torch.bool)
    others[2] = False
    assert not kv[0, :, others].any()
    out = torch.full((20,), 7, dtype=torch.int64, device="cuda")
    rc = _hip.lib().actkv_slot_map(table.data_ptr(), 2, 3, 6, bs, out.data_ptr(), _hip.stream(kv.device))
    _hip.check(rc, "actkv_slot_map")
    assert out.cpu().tolist() == [11, 36, 37, 38, 39, -1] + [7] * 14
