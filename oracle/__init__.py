"""CPU oracle for the routed sparse path — TEST INFRASTRUCTURE ONLY.

A CPU restatement (PyTorch CPU ops and plain Python) of the reference
algorithms of kreasof-ai/foveal-sparse-indexer for the hot path: routing
(foveal_indexer/core.py), the block-sparse Pattention MLP
(foveal_indexer/foveal_pattention.py, pattention_triton.py), foveal decode
attention (foveal_indexer/attention.py) and block-sparse linear / 2-D tiled
matmul (foveal_indexer/block_matmul.py, triton_ops.py).  Each function cites
the reference lines it restates.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker or the CPU baseline.  The product
(foveal-sparse-indexer_amd/) never imports it and has no CPU path.

How each function is pinned (see tests/test_oracle_*.py):
  routing.masked_probs        known answer (reference tests/test_indexer.py:10-18) + fp64 closed form
  routing.select_route        known answers (tests/test_indexer.py:20-61) + pure-Python brute force
                              (oracle/brute.py) on tiny rows + closed-form special cases
  routing.cosine_scores_f32   closed form: cos(q, k) / sqrt(d) in fp64
  routing.mlp_pooled_route    fp64 recomputation of the pooled score + brute-force top-k
  routing.decode_route        brute force per sequence + reference invariant (tests/test_attention.py:37-62)
  indexer.*                   brute-force loops (rms_norm, block pooling, additive context) and
                              the cos / sqrt(d) closed form
  indexer.distillation_loss   pure-Python brute force (oracle/brute.py), closed forms (teacher =
                              student softmax -> entropy; zero teacher -> uniform target), gradcheck
  pattention.*                identity with dense SwiGLU in fp64 when every block is active, and
                              masked-dense SwiGLU for any active set
  attention.decode_attention_f64
                              single-token and equal-score closed forms, torch SDPA in fp64
  attention.DecodeStepOracle  page pooling against an fp64 recomputation
  blocksparse.*               brute-force loops, the dense special case (F.linear), tile ids and
                              row groups, closed forms of the eval block selection
"""
