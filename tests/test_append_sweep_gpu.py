"""Device append (actkv_append through PagedKVCache.append / append_batch) over a seeded random
sweep, against the oracle's paged cache model, bit-exact (paged.py:67-85).

Each case draws the cache dtype (bf16, fp16, fp32), Hkv 1/2/3/8, head_dim 4/12/40/64/128,
block 4/8/16/32/64, 1-3 layers and a shuffled free stack, then 6 steps, each either one
request's append or an append_batch over several requests, with 0-300 tokens per request,
k and v each of a random source dtype (fp32, bf16, fp16), sometimes a strided view into a wider
tensor.  The sources carry rounding edge cases (bf16 halfway points, fp16 overflow and
subnormals).  After every step the cache bytes, free stack, tables and seq_used equal the
model's after the same appends of the sources converted by torch on the CPU.
"""
import math
import random

import pytest
import torch

from actkv.paged import PagedKVCache  # noqa: F401  (the cache under test, built by _pair)
from test_append_gpu import _bits_np, _pair, _same, _source

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def _src(shape, dtype, g, strided, rnd):
    if not strided:
        return _source(shape, dtype, g)
    pad = rnd.randint(1, 5)
    wide = _source(shape[:-1] + (shape[-1] + pad,), dtype, g)
    off = rnd.randint(0, pad)
    return wide[..., off: off + shape[-1]]


@pytest.mark.parametrize("seed", range(32))
def test_random_appends_match_the_model(seed):
    rnd = random.Random(4000 + seed)
    kv_dtype = rnd.choice(DTYPES)
    hkv, d = rnd.choice([1, 2, 3, 8]), rnd.choice([4, 12, 40, 64, 128])
    bs, layers = rnd.choice([4, 8, 16, 32, 64]), rnd.randint(1, 3)
    steps = []
    for _ in range(6):
        reqs = rnd.sample(range(5), rnd.randint(1, 4)) if rnd.random() < 0.5 else [rnd.randrange(5)]
        steps.append((reqs, [rnd.choice([0, 1, rnd.randint(2, 40), rnd.randint(41, 300)]) for _ in reqs],
                      rnd.choice(DTYPES), rnd.choice(DTYPES), rnd.random() < 0.3))
    need = {}
    for reqs, counts, *_ in steps:
        for r, c in zip(reqs, counts):
            need[r] = need.get(r, 0) + c
    nb = sum(math.ceil(n / bs) for n in need.values()) + 4
    print(f"case {seed}: {kv_dtype} Hkv {hkv} D {d} bs {bs} L {layers} steps {steps}", flush=True)
    cache, model, g = _pair(nb, bs, hkv, d, layers, kv_dtype, seed)
    for reqs, counts, kd, vd, strided in steps:
        n = sum(counts)
        k = _src((layers, n, hkv, d), kd, g, strided, rnd)
        v = _src((layers, n, hkv, d), vd, g, strided, rnd)
        if len(reqs) == 1:
            cache.append(reqs[0], k.cuda(), v.cuda())
        else:
            cache.append_batch(reqs, k.cuda(), v.cuda(), counts)
        o = 0
        for r, c in zip(reqs, counts):
            model.append(r, _bits_np(k[:, o: o + c].to(kv_dtype)), _bits_np(v[:, o: o + c].to(kv_dtype)))
            o += c
        _same(cache, model)
