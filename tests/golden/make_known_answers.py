"""Writes known_answers.json: the known answers of the reference's own tests for this path, as
data (inputs and expected outputs).  The expected outputs are the values those tests assert;
the inputs are the ones they build (random inputs are drawn here from the seeds given and
stored as explicit values).  Nothing here imports or runs the reference.

    python tests/golden/make_known_answers.py

Cases:
- keep_mask_head_reduce: tests/test_kernels.py:178-183 (mean vs max over KV heads, budget 1).
- evict_protected_and_hot: tests/test_kernels.py:157-168 (3 protected + the 4 hot tokens kept
  out of 70; the stored scores are 0.1 * uniform plus 1.0 at the hot positions).
- top_p_nucleus: tests/test_algorithms.py:16-19 (0.5 + 0.3 < 0.9 needs 0.15 too).
- lrfu_two_rounds: tests/test_algorithms.py:22-34 (Algorithm 1: decay 0.5, top-p 0.9).
- lrfu_round_without_action: tests/test_algorithms.py:37-46 (a round with no action region
  only decays).
- lrfu_intermittent_entry: tests/test_algorithms.py:49-60 (an entry hot a round ago survives
  one quiet round: keep indices [0, 3] of 5 with budget 2).
"""
import json
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def build():
    scores = torch.zeros(2, 2, 4)
    scores[0, 0, 1] = 1.0
    scores[:, :, 2] = 0.3
    keep_mask_head_reduce = {
        "cite": "tests/test_kernels.py:178-183",
        "scores": scores.tolist(), "seq_used": 4, "budget": 1,
        "expected": {"mean": [False, False, True, False], "max": [False, True, False, False]},
    }
    hot = [5, 17, 40, 69]
    ev = 0.1 * torch.rand(2, 2, 70, generator=torch.Generator().manual_seed(3))
    ev[..., hot] += 1.0
    evict_protected_and_hot = {
        "cite": "tests/test_kernels.py:157-168",
        "layers": 2, "kv_heads": 2, "head_dim": 16, "block_size": 16, "tokens": 70,
        "scores": ev.tolist(), "budget": 4, "protected": 3,
        "expected": {"sorted_perm": [0, 1, 2, *hot], "seq_used": 7, "blocks": 1},
    }
    top_p_nucleus = {
        "cite": "tests/test_algorithms.py:16-19",
        "scores": [0.5, 0.05, 0.3, 0.15, 0.0], "top_p": 0.9,
        "expected": [True, False, True, True, False],
    }
    lrfu_two_rounds = {
        "cite": "tests/test_algorithms.py:22-34",
        "decay": 0.5, "top_p": 0.9,
        "rounds": [{"act": [0.05, 0.05, 0.8, 0.1], "seq_used": 4, "active": True,
                    "expected_ks": [0.0, 0.0, 0.8, 0.1]},
                   {"act": [0.0, 0.0, 0.0, 0.05, 0.95, 0.0], "seq_used": 6, "active": True,
                    "expected_ks": [0.0, 0.0, 0.4, 0.05, 0.95, 0.0]}],
    }
    lrfu_round_without_action = {
        "cite": "tests/test_algorithms.py:37-46",
        "decay": 0.5, "top_p": 0.9,
        "rounds": [{"act": [0.05, 0.05, 0.8, 0.1], "seq_used": 4, "active": True,
                    "expected_ks": [0.0, 0.0, 0.8, 0.1]},
                   {"act": [0.0] * 6, "seq_used": 6, "active": False,
                    "expected_ks": [0.0, 0.0, 0.4, 0.05, 0.0, 0.0]}],
    }
    lrfu_intermittent_entry = {
        "cite": "tests/test_algorithms.py:49-60",
        "decay": 0.5, "top_p": 0.9,
        "rounds": [{"act": [0.9, 0.1, 0.0], "seq_used": 3, "active": True},
                   {"act": [0.0, 0.2, 0.0, 0.8, 0.0], "seq_used": 5, "active": True}],
        "budget": 2, "expected_keep": [0, 3],
    }
    return {"keep_mask_head_reduce": keep_mask_head_reduce,
            "evict_protected_and_hot": evict_protected_and_hot,
            "top_p_nucleus": top_p_nucleus,
            "lrfu_two_rounds": lrfu_two_rounds,
            "lrfu_round_without_action": lrfu_round_without_action,
            "lrfu_intermittent_entry": lrfu_intermittent_entry}


if __name__ == "__main__":
    with open(os.path.join(HERE, "known_answers.json"), "w") as f:
        json.dump(build(), f, indent=1)
        f.write("\n")
