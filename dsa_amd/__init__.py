"""MI355X (gfx950) Lightning-Indexer decode path.

Dense 64-head x 128-dim indexer scoring, exact stable top-K, block summaries
and temporal/progressive pruning, computed by hand-written HIP kernels in
``libdsa_amd.so`` behind the C ABI of ``include/dsa_amd.h``.  The modules keep
the names of the reference package ``temporal_dsa``:

  progressive_kernel  dense / H8 / masked / progressive scoring
  metrics             stable_topk, topk, topk_recall
  verifier_scoring    score_head_sparse, score_dim_sparse, normalized_hadamard,
                      fake_symmetric_quantize, dynamic_head_indices
  verifier            live two-path verifier step, dim sketches, step metrics
  approx              device own-trajectory policy state and step
  sidecar             LightningIndexerSidecar encoders and score_encoded
  certified           block_key_norms, temporal_score_radius
  temporal            device temporal pruning (seed, hot-first, running top-K)
"""

from ._lib import load as load_library

__all__ = ["load_library"]
