"""Parity pins that depend on torch's CPU arithmetic, checked on the host the GPU tests run on.

1. Keep mask: the device reduces each token's scores over KV heads and then layers in the
   float32 order of torch's CPU `mean` (actkv/paged.py:34-37).  The keys kernel leaves each
   token's order-preserving uint32 key in the keep workspace; decoded, it must equal this
   host's `scores.mean(-2).reshape(-1, S).mean(0)` bit for bit, for the shapes whose order
   tests/test_oracle.py pins against the documented cascade.
2. LRFU nucleus: the device takes equal scores lowest index first and rounds a float64 total
   to float32; the reference (actkv/eviction.py:36-50) sorts without a stable order and sums
   in float32.  Against that reference form every differing entry must be explained: it is
   tied with the reference's boundary value, or its rank lies between the nucleus sizes the
   two totals give.
"""
import numpy as np
import pytest
import torch

from actkv import _hip
from actkv.kernels.lrfu import lrfu_update
from actkv.paged import keep_mask_from_scores
from oracle import reference as ref

pytestmark = pytest.mark.gpu


def _decode_keys(keys: np.ndarray) -> np.ndarray:
    """float32 values of the device's order-preserving keys (key 0 marks a protected token)."""
    k = keys.astype(np.uint32)
    bits = np.where(k >= 0x80000000, k & 0x7FFFFFFF, ~k).astype(np.uint32)
    return bits.view(np.float32)


@pytest.mark.parametrize("L,H,S,W", [(36, 8, 4096, 4096), (36, 8, 1000, 1024), (1, 8, 333, 333), (20, 8, 640, 700),
                                     (40, 16, 97, 128), (3, 3, 65, 65), (200, 8, 256, 256), (36, 32, 70, 96)])
def test_device_layer_mean_is_this_hosts_torch_mean(L, H, S, W):
    g = torch.Generator().manual_seed(L + S)
    x = (torch.rand(L, H, W, generator=g) * torch.exp(torch.randn(L, H, W, generator=g) * 3)).float()
    want = x[..., :S].mean(-2).reshape(-1, S).mean(0)          # torch's CPU mean on this host
    xd = x.to("cuda")
    keep_mask_from_scores(xd[..., :S], S, budget=min(10, S), protected=0)
    # the call's cached workspace (per device: keyed by the tensors' device), keys first
    ws = _hip.workspace(xd.device, _hip.WS_KEEP_MASK, 1, S)
    keys = ws[: 4 * S].cpu().numpy().view(np.uint32)
    got = _decode_keys(keys)
    print(f"L={L} H={H} S={S}: cpu capability {torch.backends.cpu.get_cpu_capability()}, "
          f"{torch.get_num_threads()} threads", flush=True)
    assert np.array_equal(got.view(np.uint32), want.numpy().view(np.uint32)), \
        f"{int((got != want.numpy()).sum())} of {S} layer means differ from this host's torch mean"


def _explain(a: torch.Tensor, dev_hit: torch.Tensor, p: float):
    """Entries where the device nucleus differs from the reference form, each classified; an
    unexplained entry fails.  Returns (differing entries, by ties, by totals)."""
    want = ref.top_p_mask(a, p, stable=False, total64=False)
    diff = torch.nonzero(want != dev_hit).flatten()
    if diff.numel() == 0:
        return 0, 0, 0
    vals, order = torch.sort(a, descending=True, stable=True)
    csum = torch.cumsum(vals, 0)                                   # float64 sums stored as float32
    rank = torch.empty_like(order)
    rank[order] = torch.arange(order.numel())
    n32 = min(int(torch.searchsorted(csum, p * a.sum()).item()) + 1, a.numel())
    n64 = min(int(torch.searchsorted(csum, p * a.double().sum().float()).item()) + 1, a.numel())
    boundary = vals[n32 - 1]
    ties = totals = 0
    for i in diff.tolist():
        if float(a[i]) == float(boundary):
            ties += 1
        elif min(n32, n64) <= int(rank[i]) < max(n32, n64):
            totals += 1
        else:
            raise AssertionError(f"entry {i} (value {float(a[i])!r}, rank {int(rank[i])}): nucleus sizes "
                                 f"{n32} (float32 total) / {n64} (float64 total), boundary {float(boundary)!r}")
    return diff.numel(), ties, totals


@pytest.mark.parametrize("seed", range(12))
def test_lrfu_nucleus_against_the_reference_form(seed):
    rng = np.random.default_rng(seed)
    L, H, R = 4, 8, 3
    seqs = [int(rng.integers(200, 20000)) for _ in range(R)]
    W = max(seqs) + 16
    p = float(rng.choice([0.5, 0.8, 0.9, 0.95, 0.99]))
    g = torch.Generator().manual_seed(seed)
    kind = seed % 3
    if kind == 0:        # heavy-tailed means of probabilities
        scores = (torch.rand(L, R, H, W, generator=g) ** 8) * 1e-2
    elif kind == 1:      # few distinct values: many ties at the boundary
        scores = torch.randint(0, 6, (L, R, H, W), generator=g).float() * 1e-3
    else:                # uniform
        scores = torch.rand(L, R, H, W, generator=g)
    scores[torch.rand(L, R, H, W, generator=g) < 0.05] = 0.0
    ks = torch.zeros(L, R, W, device="cuda")
    hits = lrfu_update(scores.cuda(), ks, seqs, [4] * R, True, 0.5, p, return_hits=True).cpu()
    n = t = o = 0
    for r, S in enumerate(seqs):
        act = ref.paged_lrfu_act(scores[:, r], S)
        for l in range(L):
            d, ti, to = _explain(act[l, 4:S], hits[l, r, 4:S], p)
            n, t, o = n + d, t + ti, o + to
    print(f"seed {seed}: {n} entries differ from the reference form ({t} tied at the boundary, "
          f"{o} between the two totals' nucleus sizes)", flush=True)
