"""CPU oracle for the batched linear-bound-propagation path.

TEST INFRASTRUCTURE ONLY.  This package restates, op for op in PyTorch on
the CPU, the reference functions the HIP library replaces, so tests can check
the GPU results against it and ``bench.py`` can time it as the CPU baseline.
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import it; the product package never does.

Modules:
  ref_bound  -- slopes, IBP, zonotope forward, CROWN backward and
                concretization, CROWN intermediate bounds, alpha-CROWN,
                beta split term (verify_zono_bnb.py, verify_milp.py)
  ref_bab    -- closure, halfspace clipping, branching, bisection,
                compaction, LIFO chunk worklist, input-split driver
                (verify_graph.py)

Pinning: every function is checked by tests/test_oracle_*.py against closed
forms, the reference's own known-answer tests, sampled ground truth, brute
force on tiny inputs, or golden vectors (tests/golden/).
"""
