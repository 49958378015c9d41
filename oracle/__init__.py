"""CPU oracle of the tree-verification path — TEST INFRASTRUCTURE ONLY.

Nothing in the product (the diffspec_mi355x package, libdsv.so) imports,
links or runs anything here.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` use this package, and only as
the checker / the timed CPU reference, never as the thing measured or shipped.

Modules
  attention     numpy float64 closed forms of the attention path (A1-A8)
  accept        restatement of the greedy walk (draft/tree_verification.py:100-182),
                the typical (posterior) walk and an independent brute force
  bundles       restatement of the bundle scheduler (core/bundle_scheduler.py:42-171)
                and the query packing order built from it
  sampling      the sampling branch of verify_new (draft/tree_verification.py:103-106
                with the warpers of :15-32) as a seeded counter-based Gumbel-max draw
  ref_cpu_path  the reference's own torch CPU op sequence (repeat_kv -> prefix
                matmul/softmax/logsumexp -> naive tree -> sigmoid merge -> walk),
                timed as the CPU baseline

Pinning (what each function is checked against, besides the GPU):
  masked_attention      brute force per row, special cases (constant V, q = 0,
                        planted key, chain tree = causal, star tree), split
                        invariance of the LSE merge — tests/test_oracle_attention.py
  ancestor_mask         brute-force walk and the bitmask recurrence
  greedy_walk           brute force over root paths, hand-made trees (ties,
                        full accept, root only) — tests/test_oracle_accept.py
  bundles.packing_order the reference's scheduler vectors, hand-worked orders,
                        invariants on generated trees — tests/test_oracle_bundles.py
  sampling              Random123's known-answer vectors of Philox4x32-10 (the
                        counter RNG), numpy's log/exp2
                        (the deterministic ln / 2^x), transformers' own warpers on
                        committed fixture rows (tests/golden/sampling_warpers.json),
                        an independent float nucleus, chi-square of the draws
                        against the softmax — tests/test_oracle_sampling.py
  typical_walk          closed forms of the entropy (uniform, one-hot) and the
                        greedy/typical relation on planted cases.  The reference
                        has no typical acceptance: parity with the reference is
                        UNPINNED for this function by construction.
"""
