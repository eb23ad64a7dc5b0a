"""CPU oracle for the kernel_library hot path -- TEST INFRASTRUCTURE ONLY.

Nothing in the product (``nki-autotune_amd/``) imports this package.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may use it, and only as the checker (or, for bench, as the
timed CPU baseline), never as the thing measured on the GPU.

It restates the reference's numerics in numpy:

* ``bf16``       -- round-to-nearest-even float32 -> bfloat16 (the reference
                    casts through ml_dtypes, types.py:17-30; absent here).
* ``inputs``     -- seeded input generation in signature order
                    (reference autotune/src/autotune/runner/benchmark.py:156-169).
* ``matmul``     -- ``lhs_T.T @ rhs`` closed form (the reference golden,
                    examples/tune_matmul_lhsT_rhs.py:165), a brute-force fp64
                    loop, and a tile-faithful emulation of the hand kernel's
                    loop nest (kernel_library/matmul/lhsT_rhs/
                    kernel_hand_90.92mfu.py:72-131).
* ``rmsnorm``    -- two-pass rmsnorm_matmul closed form and the online
                    "Algorithm 4" emulation (kernel_library/rmsnorm_matmul/
                    kernel_hand_online.py:1-26, 93-192, 198-353).
* ``metrics``    -- the reference's error report (kernel_transforms.py:594-597).

Parity pins (tests/test_oracle.py, tests/test_oracle_mutations.py): every
function above is checked against at least one of: the reference's own
procedures (seed-0 N(0,1) at 128^3 atol=rtol=1e-4, test/ops/
test_direct_numpy_call.py:32-38; the 256x256x512 small fixture,
test/transforms/_fixtures.py:36-59), an independent brute-force loop, a
textbook identity (lhs_T = I, W = I, linearity, K-split associativity,
K-permutation invariance, scale invariance, zero rows), torch's own bf16
rounding, and committed golden vectors (tests/golden/).  The bf16 hardware
output of the reference is never compared by the reference itself
(benchmark.py:135,146-153), so bf16 device parity is pinned by the benchmark's
contract (max-rel <= 1e-2 against the fp32/fp64 closed form) -- no oracle
function is left "parity unpinned".
"""
