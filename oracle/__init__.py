"""ORACLE: CPU restatement of the SeoulKV4 sparse decode step.

Test infrastructure only.  ``tests/``, ``__graft_entry__.smoke()`` and the
CPU-baseline leg of ``bench.py`` may import it, and only as the checker; the
product path (``seoulkv_amd``) never imports, links or runs anything here and
fails loudly when its HIP library is missing.

Parity status per function (what pins each, besides GPU parity):
* ``arith.fixed_point`` / ``exact_dot`` / ``to_f32`` / ``sqrt_rne_f32`` —
  pinned by exact rational arithmetic (``fractions``) and ``math.isqrt``
  brute force in ``tests/test_oracle_arith.py``.
* ``decode.key_codec`` — closed form of ``_codecs/keys.py:16-26``; pinned by
  an independent torch evaluation of that formula and bucket-boundary checks.
* ``decode.coarse`` / ``fine_scores`` / ``scores_*bit`` — pinned by float64
  evaluation of the reference's decoded operands (within one BF16 ulp plus
  fixed-point truncation) and by exact Fraction evaluation on small cases.
* ``decode.thresholds`` / ``survivor_masks`` / ``fine_select`` /
  ``top_tokens`` — pinned by brute-force full sorts and the reference's
  invariants (every head keeps >= P survivors; selected within survivors).
* ``decode.pool`` — pinned against a literal restatement of the reference's
  ``encounter_union`` loop and the ``expand_lists`` sorted-set identity.
* ``decode.sdpa`` — pinned against ``torch.nn.functional.scaled_dot_product_attention``.
* The Tensix FPU accumulation order and packer rounding of the reference are
  third-party (TT-Metal 0.77.0) and cannot run here: the canonical arithmetic
  in ``arith`` replaces them, so bit-exactness is against that definition.
"""
