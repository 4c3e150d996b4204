"""The oracle against the known answers of the reference's own tests, stored as data in
tests/golden/known_answers.json (written by tests/golden/make_known_answers.py; each case
cites the reference test it comes from).  tests/test_golden_gpu.py holds the device path to
the same file."""
import json
import math
import os

import numpy as np
import torch

from oracle import reference as ref

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")))


def test_fixture_matches_its_generator():
    """The committed file is what the committed script writes."""
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "make_known_answers", os.path.join(os.path.dirname(__file__), "golden", "make_known_answers.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    assert json.loads(json.dumps(mod.build())) == GOLDEN


def test_keep_mask_head_reduce():
    c = GOLDEN["keep_mask_head_reduce"]
    s = torch.tensor(c["scores"])
    for how, want in c["expected"].items():
        assert ref.keep_mask_from_scores(s, c["seq_used"], budget=c["budget"], head_reduce=how).tolist() == want


def test_evict_protected_and_hot():
    c = GOLDEN["evict_protected_and_hot"]
    n, bs = c["tokens"], c["block_size"]
    m = ref.PagedCacheModel(math.ceil(n / bs) + 2, bs, c["kv_heads"], c["head_dim"], c["layers"])
    g = torch.Generator().manual_seed(0)
    k = torch.randn(c["layers"], n, c["kv_heads"], c["head_dim"], generator=g).to(torch.float16)
    m.append(0, k.view(torch.int16).numpy().view(np.uint16), k.view(torch.int16).numpy().view(np.uint16))
    perm = m.evict(0, torch.tensor(c["scores"]), budget=c["budget"], protected=c["protected"])
    want = c["expected"]
    assert sorted(perm.tolist()) == want["sorted_perm"]
    assert m.seq_used[0] == want["seq_used"] and len(m.tables[0]) == want["blocks"]


def test_top_p_nucleus():
    c = GOLDEN["top_p_nucleus"]
    s = torch.tensor(c["scores"])
    assert ref.top_p_mask(s, c["top_p"]).tolist() == c["expected"]
    assert ref.top_p_mask(s, c["top_p"], stable=True, total64=True).tolist() == c["expected"]


def _lrfu(c):
    ks = torch.zeros(0)
    for rd in c["rounds"]:
        S = rd["seq_used"]
        ks = torch.cat([ks, torch.zeros(S - ks.numel())])
        ref.lrfu_update(ks, torch.tensor(rd["act"]), S, 0, c["decay"], c["top_p"], active=rd["active"])
        if "expected_ks" in rd:
            torch.testing.assert_close(ks, torch.tensor(rd["expected_ks"]))
    return ks


def test_lrfu_two_rounds():
    _lrfu(GOLDEN["lrfu_two_rounds"])


def test_lrfu_round_without_action():
    _lrfu(GOLDEN["lrfu_round_without_action"])


def test_lrfu_intermittent_entry():
    c = GOLDEN["lrfu_intermittent_entry"]
    ks = _lrfu(c)
    keep = ref.keep_mask_from_scores(ks, ks.numel(), budget=c["budget"])
    assert torch.nonzero(keep).flatten().tolist() == c["expected_keep"]
