"""Scoring parity with one MFMA kernel forced for every query-row count (run by
test_scoring_forced_gpu.py in a child process whose ACTKV_SCORE_KERNEL selects the kernel: the
library reads it once per process).  Each case: 3 requests, one layer, causal limits or none, a
partial query count per request, running means with earlier counts; against the oracle's fold
(lse_attn.py:63-78) at rtol 1e-3."""
import math
import os
import sys

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
for p in (ROOT, os.path.join(ROOT, "actkv-open_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

import torch  # noqa: E402

from actkv.kernels.lse_attn import action_scores  # noqa: E402
from actkv.paged import PagedKVCache  # noqa: E402
from oracle import reference as ref  # noqa: E402

# (dtype, hq, hkv, n_q, block, causal): 32..512 query rows over groups 4, 2 and 1
CASES = [
    (torch.bfloat16, 32, 8, 8, 16, True), (torch.bfloat16, 32, 8, 16, 16, False),
    (torch.float16, 32, 8, 24, 32, True), (torch.bfloat16, 32, 8, 32, 16, True),
    (torch.bfloat16, 32, 8, 40, 16, False), (torch.float16, 32, 8, 64, 16, True),
    (torch.bfloat16, 32, 8, 80, 64, True), (torch.bfloat16, 32, 8, 96, 16, False),
    (torch.bfloat16, 32, 8, 112, 16, True), (torch.float16, 32, 8, 128, 16, False),
    (torch.bfloat16, 16, 8, 40, 16, True), (torch.float16, 16, 8, 100, 16, False),
    (torch.bfloat16, 16, 8, 200, 32, True), (torch.bfloat16, 8, 8, 100, 16, True),
    (torch.float16, 8, 8, 300, 16, False), (torch.bfloat16, 8, 8, 450, 16, True),
]


def run_case(i, dtype, hq, hkv, n_q, bs, causal):
    lens = [700, 90, 1500]
    g = torch.Generator().manual_seed(100 + i)
    nb = sum(math.ceil(n / bs) for n in lens) + 5
    cache = PagedKVCache(nb, bs, hkv, 128, n_layers=1, dtype=dtype, device="cuda")
    cache.free = torch.randperm(nb, generator=g).tolist()
    for r, n in enumerate(lens):
        cache.append(r, torch.randn(1, n, hkv, 128, generator=g).to(dtype).cuda(),
                     torch.randn(1, n, hkv, 128, generator=g).to(dtype).cuda())
    reqs = [0, 1, 2]
    bt, seq = cache.block_table(reqs), cache.seq_tensor(reqs)
    width = bt.shape[1] * bs
    q = torch.randn(3, n_q, hq, 128, generator=g).to(dtype)
    kv0 = cache.kv[0].cpu()
    tables = [cache.tables[r] for r in reqs]
    lse = torch.stack([ref.decode_lse(q[:, n], kv0, tables, lens) for n in range(n_q)], 1)
    kv_len = (torch.stack([torch.randint(1, s + 1, (n_q,), generator=g) for s in lens]).to(torch.int32)
              if causal else None)
    n_valid = torch.tensor([n_q, max(1, n_q // 3), n_q - 1], dtype=torch.int32)
    out0 = torch.rand(3, hkv, width, generator=g)
    n0 = torch.tensor([0, 5, 2], dtype=torch.int32)
    out_k, n_k = out0.cuda(), n0.cuda()
    action_scores(q.cuda(), cache.kv[0], bt, seq, lse.cuda(), out_k, n_k, n_valid=n_valid.cuda(),
                  kv_len=None if kv_len is None else kv_len.cuda())
    out_o, n_o = out0.clone(), n0.clone()
    ref.action_scores_nfold(q, kv0, tables, lens, lse, out_o, n_o, n_valid=n_valid, kv_len=kv_len)
    torch.testing.assert_close(out_k.cpu(), out_o, rtol=1e-3, atol=1e-6)
    assert torch.equal(n_k.cpu(), n_o)


if __name__ == "__main__":
    kernel = os.environ.get("ACTKV_SCORE_KERNEL", "auto")
    for i, c in enumerate(CASES):
        print(f"{kernel}: case {i} {c}", flush=True)
        run_case(i, *c)
    print(f"{kernel}: {len(CASES)} cases match the oracle", flush=True)
