"""The oracle: a CPU restatement of the reference's PyTorch bf16 path for the hot path (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this package, and only as the checker (or
as the timed CPU baseline). The product path (strix-halo-maxx_amd/) never imports it.

Each function cites the reference file:line it restates. The reference's own code cannot run here (moondream2 and
TAPNext weights/models are remote or external; its HIP kernels target gfx1151), so "matches the reference" means
"matches this restatement". How each function is pinned is stated in its docstring:
  * md2_vision:  LayerNorm, GELU-tanh, SDPA, Linear pinned by closed forms / fp64 brute force (tests/test_oracle_*.py)
  * md2_text:    rope pinned against the explicit rotation (fused.py:53-58 restated), mask against the closed form
                 (md2fast.py:132-136), greedy loop by argmax identity; freqs_cis theta=10000 is an assumption
                 (parity unpinned for the theta value itself)
  * trecvit:     RMSNorm / LN / GELU against pack8.py closed forms; RG-LRU against its invariants (first frame, a -> 1,
                 fixed point, associative-scan == sequential in fp64)
"""
