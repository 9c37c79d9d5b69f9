"""CPU restatement of the reference's block-sparse attention hot path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this package, and only as the
checker or the reported CPU baseline.  The product (``dit_sparse_atten_amd``)
never imports it and has no CPU fallback.

The reference is Python (PyTorch + FlexAttention + Triton), so there is no C
or C++ reference source to compile into an ``oracle/_ref`` library; the
restatement is numpy (fp32 / fp64 / exact integers) and plain Python loops.

Modules, the reference code each follows, and what pins each function
(tests/test_oracle_*.py; golden fixtures written by tests/golden/make_golden.py
from the reference imported in the build container):

  attention    block_sparse_attention: masked softmax closed form in fp64
               (flex.py:379-399, sparse.py:670-751).  Pinned by: full route ==
               torch SDPA; equality with the reference's own sparse_chunk
               outputs on config 0 (sparse_config0.npz).
  route        sample_indices (flex.py:221-231): known answers (offsets
               4, 12, ..., 124; partial blocks).
               sampled_block_mass (flex.py:205-251): reference golden
               (sampled_mass.npz checksums), S = block => exact block mass.
               persistence_prior (flex.py:535-541): reference golden
               (sampled_route.npz), dyadic closed form.
               top_mass_route (flex.py:83-94 == sparse.py:171-181): reference
               golden (top_mass_route.npz, ties compared as value multisets
               because torch's CPU argsort is unstable), brute force over all
               prefixes with exact rationals, planted-mistake checks.
               first_frame_sink (flex.py:550-566), pack_rows
               (layout_ops.py:128-151), to_csr (flex.py:275-338), route_keep /
               dense_dispatch (flex.py:473-493): known answers from the
               reference's tests, stable argsort, round trips.
  exact        dense_lse, exact_block_mass(_rows), exact_route (flex.py:96-106,
               158-202, 254-272): the reference's own identities (full sampling
               S = block equals exact / block, test_flex_backend.py:43-53;
               explicit padded softmax, test_flex_backend.py:62-76), rows summing
               to the valid query count, planted mistakes.
  routing      frontier_mask, best_targets, select_fixed_budget,
               directional_budget_update (routing.py:10-168): reference golden
               (routing.npz: two frontiers and three directional updates on the
               720p neighbour table, bit-exact), the reference's known answers
               (test_directional_routing.py), invariants, planted mistakes.
  spatial      morton_code, choose_microtile, spatial_layout (spatial.py:14-183)
               and sparse_tile_shape / tile_major_permutation (sparse.py:51-138):
               reference golden (spatial_layout.npz, the full 57,600-token
               permutation and neighbour table), known answers, bijection.
  dropout      philox4x32_10, keep_mask, dropout_attention (SDPA's dropout as
               DenseBackend hands it on, dense.py:40-47; the mask from
               Philox4x32-10, Salmon et al. 2011): Random123's three
               known-answer vectors, keep fraction 1 - p, a planted wrong
               multiplier, dropout_p -> 0 equal to the attention closed form.
  sparse_path  group_indices, sparse_chunk, dense_route, SparsePathCase
               (sparse.py:184-233, 376-406, 670-751, 794-930): reference golden
               on config 0 (bootstrap route, mass, outputs, one sparse step).

No function of the oracle is left without such a check.
"""
