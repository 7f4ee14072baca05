"""CPU oracle for the full-attention hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in ``supersonic_amd`` imports this package;
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and always as the checker or the timed CPU baseline, never
as the product path.  The product path is the HIP library and fails loudly when
it is missing.

Modules:
  attn_oracle  torch fp32 restatement of the reference's attention semantics
               (QK RMSNorm, partial RoPE, causal / decode GQA attention, gate,
               the prefill chain and the fused decode step).
  fp8_codec    numpy restatement of both e4m3 codecs: OCP e4m3fn (what gfx950
               converts in hardware) and the reference's hand-rolled codec with
               its subnormal constant and exponent-14 clamp.
  brute        float64 pure-python/numpy brute force used to pin attn_oracle on
               tiny shapes (an independent implementation, not a retype).
"""
