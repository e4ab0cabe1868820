"""CPU oracle for the batch-1 decode hot path. TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import anything from this package. The product path (the HIP extension behind ``decode``) never
routes through it; it is the checker.

Modules:
  ``spec``     model shapes, the reference's per-layer weight order, synthetic-input protocol.
  ``hf``       the reference's own arithmetic: Hugging Face Transformers ``Qwen3ForCausalLM`` on CPU
               (seeded random init, prefill, teacher-forced decode, K/V cache export).
  ``restate``  a float32 torch restatement of one decode step with bf16 rounding at exactly the
               points Transformers rounds, and an attention that follows torch's CPU flash SDPA
               (512-key blocks, bf16 probabilities, ``exp_u20``); also an all-fp32 mode that
               follows ``megakernel.cu``.
"""
