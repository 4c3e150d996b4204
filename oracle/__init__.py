"""CPU oracle for the ActKV eviction hot path -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

A restatement of the reference's algorithm (Maurya30/actkv-open: actkv/kernels/lse_attn.py,
actkv/kernels/compaction.py, actkv/paged.py) used only to compare and time against:

  * tests/ compare the HIP kernels against it on identical seeded inputs;
  * __graft_entry__.smoke() checks one small run against it;
  * bench.py's cpu_baseline leg times it on the host cores.

Nothing in the product package (actkv-open_amd/) may import, call or link anything here.

Pinning (what fixes each function independently of its own formula; see tests/test_oracle.py):
  action_scores_fold    known answer: probabilities of one query sum to 1 (tests/test_kernels.py:58-66
                        of the reference); brute force with float64 Python loops on tiny inputs;
                        running mean of N folds == arithmetic mean; GQA group sharing q and lse ==
                        single head; invariance to physical block permutation.
  action_scores_nfold   equals action_scores_fold fold by fold (same float32 operations).
  decode_lse            torch.logsumexp (library routine) in float64; checked against a direct
                        log(sum(exp)) on tiny inputs.
  keep_mask_from_scores known answers of the reference tests (paged.py semantics,
                        tests/test_kernels.py:157-183); brute-force sort on tiny inputs.
  torch_mean_emulation  bit-exact against torch's own CPU mean on random inputs (this pins the
                        summation order the device reduction follows).
  plan_compaction       brute force from the definition (pure-Python loops) on every small case;
                        invariants of tests/test_kernels.py:80-91 (disjoint, perm is a permutation
                        of the kept positions, drop = ceil(S/bs) - ceil(B/bs)).
  apply_copies          memcpy semantics; tests/test_kernels.py:94-102 shape.
  PagedCacheModel       known answers tests/test_kernels.py:122-200 (free-list stack order,
                        protected prefix survives repeated evictions).
"""
