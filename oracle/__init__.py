"""CPU oracle for the indexer hot path -- TEST INFRASTRUCTURE ONLY.

This package restates the reference algorithms (psa1582/dsa, ``temporal_dsa``)
on the CPU with numpy / torch-CPU so that the HIP kernels of ``dsa_amd`` can be
checked against them.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker or
as the timed CPU baseline.  The product package ``dsa_amd`` never imports it
and has no CPU fallback.

Modules and what pins each restatement (tests under ``tests/``):

  scores     dense / progressive / multi-query / head-sparse scores.
             Pinned by the closed form sum_h w_h max(0, q_h.k) in float64,
             explicit per-key loops on tiny inputs and the reference's test
             invariants (all-promoted == full, +inf threshold, ragged block).
  topk       stable_topk and recall.  Pinned by brute force (lexsort over
             (-value, index)) on random and tie-heavy inputs and by the
             reference's tie tests.
  replay     replay_transition / replay_trace (temporal pruning replay) with
             an extra ``wave`` parameter; wave == 1 is the reference.  Pinned
             by the reference's replay tests, hand-built cases with known
             counts, a brute-force sequential simulator, and golden vectors
             recorded from the reference under ``tests/golden/``.
  approx     initialize_state / replay_step (own-trajectory pruning).  Pinned
             by the reference's approx tests, hand cases and golden vectors.
  certified  temporal_score_radius / block_key_norms.  Pinned by the
             covering inequality on random signed-weight inputs and by
             closed forms (zero drift gives radius 0, a single head reduces to
             Cauchy-Schwarz).
"""
