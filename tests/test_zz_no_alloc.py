"""actkv_keep_mask_noalloc (the keep mask on the library's static device scratch) against
actkv_keep_mask on a caller workspace, through the C ABI: three calls in a row on one GPU,
each smaller than or different from the last, must give bit-identical keep masks and keep
bits; a call larger than the scratch is refused before any launch."""
import numpy as np
import pytest
import torch

from actkv import _hip

pytestmark = pytest.mark.gpu


def _keep(entry, scores, L, H, R, seq, budget, prot_count, prot_mask, reduce, max_seq, bs=16, ws=None):
    dev = scores.device
    keep = torch.zeros(R, max_seq, dtype=torch.bool, device=dev)
    nw = (-(-max_seq // bs) * bs + 31) // 32
    bits = torch.zeros(R, nw, dtype=torch.int32, device=dev)
    args = [scores.data_ptr(), _hip.dtype_code(scores.dtype), scores.stride(0), scores.stride(1), scores.stride(2),
            L, H, R, seq.data_ptr(), budget.data_ptr(), _hip.ptr(prot_count), _hip.ptr(prot_mask),
            0 if prot_mask is None else prot_mask.stride(0), reduce, keep.data_ptr(), keep.stride(0),
            bits.data_ptr(), bits.stride(0), bs, max_seq]
    lib = _hip.lib()
    if entry == "noalloc":
        rc = lib.actkv_keep_mask_noalloc(*args, _hip.stream(dev))
    else:
        rc = lib.actkv_keep_mask(*args, ws.data_ptr(), ws.numel(), _hip.stream(dev))
    _hip.check(rc, f"actkv_keep_mask ({entry})")
    return keep, bits


CASES = [
    # L, H, seqs, dtype, reduce, protected (count or mask)
    (36, 8, [9000, 4321, 8999], torch.float32, _hip.REDUCE_MEAN, "count"),
    (2, 4, [1000, 77], torch.float32, _hip.REDUCE_MAX, "count"),
    (3, 2, [500, 333], torch.bfloat16, _hip.REDUCE_MEAN, "mask"),
]


def test_noalloc_keep_mask_equals_the_workspace_entry_point():
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(0)
    for L, H, seqs, dtype, reduce, prot in CASES:
        R, max_seq = len(seqs), max(seqs)
        scores = torch.rand(L, R, H, max_seq, generator=g).to(dtype).to(dev)
        seq = torch.tensor(seqs, dtype=torch.int32, device=dev)
        budget = torch.tensor([s // 7 for s in seqs], dtype=torch.int32, device=dev)
        prot_count, prot_mask = None, None
        if prot == "count":
            prot_count = torch.tensor([4] * R, dtype=torch.int32, device=dev)
        else:
            prot_mask = (torch.rand(R, max_seq, generator=g) < 0.05).to(dev)
        need = int(_hip.lib().actkv_workspace_size(_hip.WS_KEEP_MASK, R, max_seq))
        ws = torch.zeros(need, dtype=torch.uint8, device=dev)
        ka, ba = _keep("workspace", scores, L, H, R, seq, budget, prot_count, prot_mask, reduce, max_seq, ws=ws)
        kb, bb = _keep("noalloc", scores, L, H, R, seq, budget, prot_count, prot_mask, reduce, max_seq)
        torch.cuda.synchronize()
        for r, s in enumerate(seqs):
            assert torch.equal(ka[r, :s], kb[r, :s]), (L, H, seqs, r)
            nw = (-(-s // 16) * 16 + 31) // 32
            assert torch.equal(ba[r, :nw], bb[r, :nw]), (L, H, seqs, r)
            kept = int(kb[r, :s].sum())
            n_prot = 4 if prot == "count" else int(prot_mask[r, :s].sum())
            assert kept == min(s, n_prot + s // 7), (L, H, seqs, r, kept)


def test_noalloc_keep_mask_refuses_a_call_larger_than_its_scratch():
    dev = torch.device("cuda:0")
    max_seq = (_hip.KEEP_MASK_SCRATCH_BYTES // 4) + 1024          # more keys than the scratch holds
    scores = torch.zeros(1, 1, 1, 16, device=dev)
    seq = torch.tensor([16], dtype=torch.int32, device=dev)
    keep = torch.zeros(1, 16, dtype=torch.bool, device=dev)
    rc = _hip.lib().actkv_keep_mask_noalloc(
        scores.data_ptr(), _hip.F32, 16, 16, 16, 1, 1, 1, seq.data_ptr(), seq.data_ptr(), None, None, 0,
        _hip.REDUCE_MEAN, keep.data_ptr(), 16, None, 0, 16, max_seq, _hip.stream(dev))
    assert rc == _hip.ERR_WORKSPACE
    assert _hip.lib().actkv_error_string(rc) == b"ACTKV_ERR_WORKSPACE"
