"""CPU oracle for the full-attention path: TEST INFRASTRUCTURE ONLY.

Nothing in this package is shipped or measured as the product.  Only the
tests, the smoke check and the benchmark's ``cpu_baseline`` leg may import it,
and there only as the checker (or, for ``cpu_baseline``, as the timed CPU
restatement of the reference's CPU path).  The product path lives in
``redshift_amd`` and fails loudly when its HIP library is missing.

Modules
-------
``attention_ref``  numpy restatement of ``tests/cpu_reference.py:6-15,55-89``
                   (fused RMSNorm + RoPE + fp16 append + causal GQA softmax +
                   sigmoid gate) and of the raw causal GQA core that the
                   reference's kernels compute (``src/kernels.cu:435-503``).
``kat``            the reference's closed-form long-context known-answer test
                   (``tests/test_cuda.py:237-273``), restated, plus the other
                   known answers that pin the oracle (RoPE, RMSNorm, fp16).

Pinning status (what checks each function, see tests/test_oracle.py):
  half            IEEE binary16 bit patterns (RNE, ties-to-even, overflow).
  sigmoid         closed form values.
  rmsnorm         constant-vector closed form; order RMS -> gamma -> RoPE
                  pinned by the one-hot RoPE KAT with non-uniform gamma.
  rope            one-hot closed form (rotate-half pairs (i, i+32), base 1e7).
  fused_attention closed-form long-context KAT at positions 2047 (T=3),
                  32767 and 139263 (the reference's own KAT), plus the
                  grouped == sequential invariant and prefix preservation;
                  and the reference's own output on its sine-wave fixture
                  (tests/golden/fused_attention.npz), which it matches bit
                  for bit after rounding to fp32.
  gqa_attention   torch's scaled_dot_product_attention in float64 (an
                  independent library routine), brute force on tiny shapes,
                  single-key / uniform-key / causal invariants.
  gqa_attention_fp32  same checks as gqa_attention, to fp32 tolerance.
"""
