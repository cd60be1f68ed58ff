"""CPU oracle for the attention hot path -- TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference repository's algorithms for the three
covered paths (PISA HYD block-sparse attention, fixed 64-token
block-diagonal attention, exact full attention), written from the reference
sources and citing them file:line.  It is the checker of the HIP kernels:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product package never imports it and has no
CPU fallback.

Pinning (what fixes each function independently of its own formula; the
tests live in tests/test_oracle.py and tests/test_oracle_pins.py):

* layout.ordered_to_raster / tile maps -- the reference's known answer
  (packed prefix [0..7, 96..103], test_forward.py:211-224), the torch
  reshape/permute restatement of generic_pisa.py:17-52 and exact round trips.
* attention.dense_attention -- torch.nn.functional.scaled_dot_product_attention.
* attention.fixed_block_attention -- a dense softmax with a block-diagonal
  (and causal) mask (reference.py:227-241 semantics) on tiny inputs; the
  16-bit probability rounding (prob_dtype, triton_kernel.py:92-96) by a block
  whose probabilities are exactly [1/3, 2/3]: the output is bf16(1/3) resp.
  fp16(1/3), which rounding before normalising or not rounding cannot give.
* pisa.block_stats -- textbook means / covariance (float64), ||H_b||_F via
  numpy.linalg.norm, per-block-constant keys give H = 0, bf16 extrema stay
  finite (test_forward.py:172-201).
* pisa.block_stats rounding points (tests/test_oracle_pins.py) -- exact rational
  arithmetic with one fp32 rounding per step: the Triton statistics round the
  centred keys to the dtype while HYD keeps them fp32; the means mode adds
  x * fp32(1/len) with one fma per row (distinct from sum-then-scale and from
  separately rounded products).
* pisa.route_scores -- constructed inputs whose selection is fixed by
  construction: q_bar orthogonal to every k_bar selects the largest textbook
  ||H_b|| (presence and sign of the ln bias); equal ||H_b|| selects the top
  q_bar . k_bar of a known table (no transpose); centroids whose bf16 and fp32
  products rank differently pin where each path rounds (HYD: both centroids;
  generic on HYD statistics: q_bar only; Triton statistics: neither).
* pisa.topk_ascending -- brute-force ranking with explicit ties, sink and NaN.
* layout.pack_minimax_h3_qkv -- the torch.stack copies at the 12000-token
  threshold, bit for bit.
* pisa.hyd_forward / generic_forward -- exact==N equals dense attention,
  constant V returns V, per-block-constant K makes the tail exact (no
  correction) and equals dense attention, and the LSE merge equals the
  single-softmax-over-concatenation form of test_forward.py:34-104.
* pisa.reference_forward -- budget 1 == dense, constant keys per block ==
  dense, and the closed-form first-order formula of
  tests/test_pisa_attention.py:124-146.

Parity unpinned (bit level only): the summation order of the reference's
hipBLASLt bmm, Inductor-compiled FlexAttention tiles and Triton atomics cannot
be run here; those stages are compared to tolerance (bf16 atol=rtol=5e-2).
torch.topk's tie order is unspecified; this oracle fixes ties to the lowest
index, as the HIP kernel does.
"""
