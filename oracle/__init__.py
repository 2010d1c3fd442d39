"""CPU oracle for the PersistentKV paged decode engine.

TEST INFRASTRUCTURE, NOT PRODUCT CODE.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker (bench.py times it as the CPU baseline).  The engine under
``persistentkv-attention_amd/`` never imports it and fails loudly when its HIP library is
missing.

Modules and what pins each function (the tests named here hold the checks):

``attention`` (tests/test_oracle_attention.py)
  * ``gather_row`` / ``paged_decode`` — repack + fp32 SDPA, the reference's oracle
    definition.  Pinned against an fp64 brute force, a closed-form identity gather
    (contiguous pages), reversed and canonical ``(405p+17) mod 2L`` tables, the
    uniform-attention closed form (equal keys -> mean of V) and one-hot dominance.
  * ``attention_fp64`` — textbook softmax attention; pinned by the same closed forms and
    by permutation invariance.
  * ``split_partials`` / ``lse_merge`` / ``split_bounds`` — pinned by split invariance
    (every split count gives the unsplit result), the neutral state being the merge
    identity, and the C restatement (``native``) on the same inputs.

``workqueue`` (tests/test_oracle_workqueue.py)
  * split policy, cost model and router — pinned against golden vectors written by the
    reference's own functions (tests/golden/make_policy_vectors.py).
  * ``build_workqueue`` — pinned by hand-worked known answers and the partition
    invariants of the builder (tiles of non-empty items partition [0, T) in split order,
    split_offsets is the prefix sum of the row split counts including empty splits,
    rows are padded with the last reserved page).

``native`` (tests/test_oracle_native.py)
  * C restatement of the reference kernel's fp32 arithmetic and of
    ``tests/smoke_test.cu``'s CPU reference and glibc inputs; pinned against the fp64
    brute force and the reference's recorded smoke-test error magnitudes.
"""
