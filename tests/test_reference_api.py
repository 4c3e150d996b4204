"""The reference module API kept beside the HIP path (torch formulations the reference exports:
lse_attn.py:32-78, compaction.py:72-74, :109-114, and the HAS_TRITON flag its tests and
benchmark read), checked on the CPU against the oracle's restatements."""
import numpy as np
import pytest
import torch

from actkv import _hip
from actkv.kernels import compaction, lse_attn
from oracle import reference as ref


def _paged(seed, layers=1, nb=12, bs=4, hkv=2, d=8, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    kv = torch.randn(2, nb, bs, hkv, d, generator=g).to(dtype)
    perm = torch.randperm(nb, generator=g)
    table = torch.stack([perm[:6], perm[6:]]).to(torch.int32)          # two requests, 6 blocks each
    return kv, table, g


def test_flags_report_the_compiled_kernels():
    """HAS_TRITON (the reference's name) means the compiled kernels are usable: the library is
    built and a ROCm GPU is visible."""
    assert lse_attn.HAS_TRITON == lse_attn.HAS_KERNELS == _hip.available()
    assert compaction.HAS_TRITON == compaction.HAS_KERNELS == _hip.available()


def test_gather_kv_returns_rows_in_logical_order():
    kv, table, _ = _paged(0)
    for row, s in ((0, 21), (1, 7), (1, 0)):
        k, v = lse_attn.gather_kv(kv, table, s, row)
        layer = kv.unsqueeze(0)[0]
        assert torch.equal(k, ref.gather_k(layer, table[row].tolist(), s))
        assert torch.equal(v, ref.gather_v(layer, table[row].tolist(), s))


@pytest.mark.parametrize("hq", [2, 4, 8])
def test_paged_decode_attention_ref_matches_the_oracle(hq):
    kv, table, g = _paged(1)
    q = torch.randn(2, hq, 8, generator=g)
    seq = torch.tensor([21, 9], dtype=torch.int32)
    out, lse = lse_attn.paged_decode_attention_ref(q, kv, table, seq)
    out_o, lse_o = ref.paged_attention(q[:, None], kv, table.tolist(), seq.tolist())
    torch.testing.assert_close(lse, lse_o[:, 0], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(out, out_o[:, 0], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(lse, ref.decode_lse(q, kv, table.tolist(), seq.tolist()), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("hq,dtype", [(2, torch.float32), (4, torch.float16), (8, torch.bfloat16)])
def test_action_scores_ref_folds_like_the_oracle(hq, dtype):
    kv, table, g = _paged(2, dtype=dtype)
    seq = torch.tensor([23, 17], dtype=torch.int32)
    out = torch.zeros(2, 2, 24)
    out_o = out.clone()
    ns = torch.zeros(2, dtype=torch.int32)
    ns_o = ns.clone()
    for _ in range(3):                                               # three folds, running mean
        q = torch.randn(2, hq, 8, generator=g).to(dtype)
        lse = ref.decode_lse(q, kv, table.tolist(), seq.tolist())
        lse_attn.action_scores_ref(q, kv, table, seq, lse, out, ns)
        ref.action_scores_fold(q, kv, table.tolist(), seq.tolist(), lse, out_o, ns_o)
    torch.testing.assert_close(out, out_o, rtol=1e-5, atol=1e-7)
    assert ns.tolist() == ns_o.tolist() == [3, 3]
    assert float(out[0, :, 23:].abs().sum()) == 0.0 and float(out[1, :, 17:].abs().sum()) == 0.0


def test_action_scores_ref_single_head_sums_to_one():
    """Hq = Hkv and one fold: the scores are the softmax of the query, summing to 1 over the
    request's tokens (the closed form of tests/test_kernels.py:58-66)."""
    kv, table, g = _paged(3)
    q = torch.randn(2, 2, 8, generator=g)
    seq = torch.tensor([24, 13], dtype=torch.int32)
    lse = ref.decode_lse(q, kv, table.tolist(), seq.tolist())
    out = torch.zeros(2, 2, 24)
    lse_attn.action_scores_ref(q, kv, table, seq, lse, out, torch.zeros(2, dtype=torch.int32))
    torch.testing.assert_close(out[0].sum(-1), torch.ones(2), rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(out[1, :, :13].sum(-1), torch.ones(2), rtol=1e-5, atol=1e-5)


def test_apply_copies_ref_and_gather_compaction_move_whole_rows():
    rng = np.random.default_rng(4)
    kv = torch.from_numpy(rng.integers(-30000, 30000, (6, 40, 12), dtype=np.int16))
    keep = rng.random(40) < 0.4
    src, dst, _, _ = ref.plan_compaction(keep, 37, list(range(10)), 4)
    want = kv.numpy().copy()
    ref.apply_copies(want, src, dst)
    got = kv.clone()
    compaction.apply_copies_ref(got, torch.from_numpy(src), torch.from_numpy(dst))
    assert np.array_equal(got.numpy(), want)
    slots = torch.from_numpy(np.flatnonzero(keep))
    gathered = compaction.gather_compaction(kv, slots)
    assert np.array_equal(gathered.numpy(), kv.numpy()[:, keep])
    gathered[0, 0, 0] += 1                                            # a fresh buffer, not a view
    assert not np.array_equal(gathered.numpy(), kv.numpy()[:, keep])
