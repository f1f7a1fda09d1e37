"""CPU oracle of the block-FP8 MoE expert path -- TEST INFRASTRUCTURE ONLY.

A restatement, on the CPU in torch/numpy, of the reference algorithm
(als244/mlops) for the MoE path, used as the checker of the MI355X HIP kernels.
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import it. The product package ``mlops_amd`` never does.

How each function is pinned (beyond restating the reference): see the
``PINNED`` table in ``oracle.moe_oracle`` and the tests in
``tests/test_oracle.py`` -- closed forms, library routines, brute force on
tiny inputs, autograd of the closed-form losses, and invariants chosen so
that a dropped term, wrong sign or index, or transposed operand fails.
"""
