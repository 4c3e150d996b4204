"""The device path against the known answers of the reference's own tests, stored as data in
tests/golden/known_answers.json (tests/test_golden.py holds the oracle to the same file):
the keep mask and evict through actkv_keep_mask / actkv_compact, the nucleus and the LRFU
update through actkv_lrfu_update."""
import json
import math
import os

import pytest
import torch

from actkv.kernels.lrfu import lrfu_update
from actkv.paged import PagedKVCache, keep_mask_from_scores

pytestmark = pytest.mark.gpu

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")))


def test_keep_mask_head_reduce():
    c = GOLDEN["keep_mask_head_reduce"]
    s = torch.tensor(c["scores"]).cuda()
    for how, want in c["expected"].items():
        assert keep_mask_from_scores(s, c["seq_used"], budget=c["budget"], head_reduce=how).tolist() == want


def test_evict_protected_and_hot():
    c = GOLDEN["evict_protected_and_hot"]
    n, bs = c["tokens"], c["block_size"]
    cache = PagedKVCache(math.ceil(n / bs) + 2, bs, c["kv_heads"], c["head_dim"], n_layers=c["layers"],
                         dtype=torch.float16, device="cuda")
    g = torch.Generator().manual_seed(0)
    k = torch.randn(c["layers"], n, c["kv_heads"], c["head_dim"], generator=g).to(torch.float16).cuda()
    cache.append(0, k, k)
    perm = cache.evict(0, torch.tensor(c["scores"]).cuda(), budget=c["budget"], protected=c["protected"])
    want = c["expected"]
    assert sorted(perm.tolist()) == want["sorted_perm"]
    assert cache.seq_used[0] == want["seq_used"] and len(cache.tables[0]) == want["blocks"]


def test_top_p_nucleus():
    """lrfu_update's hit mask is the nucleus of the round's (head-reduced) action scores."""
    c = GOLDEN["top_p_nucleus"]
    n = len(c["scores"])
    s = torch.tensor(c["scores"]).view(1, 1, 1, n).cuda()
    ks = torch.zeros(1, 1, n, device="cuda")
    hits = lrfu_update(s, ks, n, 0, True, 0.5, c["top_p"], return_hits=True)
    assert hits[0, 0, :n].tolist() == c["expected"]


def _lrfu(c):
    W = max(rd["seq_used"] for rd in c["rounds"])
    ks = torch.zeros(1, 1, W, device="cuda")
    for rd in c["rounds"]:
        S = rd["seq_used"]
        act = torch.zeros(1, 1, 1, W)
        act[0, 0, 0, :S] = torch.tensor(rd["act"])
        lrfu_update(act.cuda(), ks, S, 0, rd["active"], c["decay"], c["top_p"])
        if "expected_ks" in rd:
            torch.testing.assert_close(ks[0, 0, :S].cpu(), torch.tensor(rd["expected_ks"]))
    return ks


def test_lrfu_two_rounds():
    _lrfu(GOLDEN["lrfu_two_rounds"])


def test_lrfu_round_without_action():
    _lrfu(GOLDEN["lrfu_round_without_action"])


def test_lrfu_intermittent_entry():
    c = GOLDEN["lrfu_intermittent_entry"]
    ks = _lrfu(c)
    S = c["rounds"][-1]["seq_used"]
    keep = keep_mask_from_scores(ks[0, 0, :S].contiguous(), S, budget=c["budget"])
    assert torch.nonzero(keep).flatten().tolist() == c["expected_keep"]
