'''CPU oracle for the Motif Chord sequence-mixing path.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped `motif` package imports this
package; only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` may import it, and only as the checker (or as the timed CPU
baseline), never as a fallback for the HIP path.

Contents (each function cites the reference file:line it restates):

- `oracle.gdn`    gated delta rule: token recurrence, chunked (WY / UT) form,
                  short causal conv + SiLU, the GatedDeltaAttention layer, and
                  varlen wrappers (independent per-sequence runs).
- `oracle.chord`  Chord GGD-biased causal softmax attention with a materialised
                  bias, the ChordAttention layer, a pure-Python brute force for
                  tiny inputs, and varlen wrappers.
- `oracle.model`  RMSNorm / GatedRMSNorm / SwiGLU, the AttnRes read, the
                  decoder block and the MotifChordModel forward used by the
                  full-model parity tests.

The restatement is written in PyTorch on the CPU (the reference path is itself
PyTorch) so every function runs in float64 for pinning and in float32 for the
CPU baseline timing.

How each function is pinned (tests/test_oracle_*.py):
- recurrence: closed-form special cases (beta=0, g=-inf reset, single-token
  outer product, orthonormal-key exact overwrite) and an independent
  matrix-product formulation on tiny inputs;
- chunked form: equality with the recurrence for C in {16, 32, 64}, ragged L,
  and split-point continuation; the triangular inverse against
  `scipy.linalg.solve_triangular`;
- Chord: pure-Python brute force on tiny inputs, reduction to
  `scaled_dot_product_attention` when the bias is constant (alpha=0 or beta=0)
  and the logit scale is 1, uniform prefix means when log_n == 0, GQA equals
  MHA with repeated K/V, decode row equals the last prefill row;
- conv: brute-force loop;
- layer / model composition: fixtures written by importing the reference once
  in the build container (tests/golden/make_layer_fixtures.py).
'''
