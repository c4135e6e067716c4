"""CPU oracle for the decision-prefill path — TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference's algorithms for this path, used solely
as the checker: by `tests/`, by `__graft_entry__.smoke()` and by the
`cpu_baseline` leg of `bench.py`. The product package `deciax_amd` never
imports it; its kernels run on the GPU or raise.

Each function cites the reference file:line it follows (paths relative to the
deciax checkout) and, where the reference has no code for a Gemma-2 semantic,
the transformers 5.15.0 Gemma-2 code it restates (`TF/` below means
`transformers/`).

Every function takes `bf16=True` to round at the reference's bf16 rounding
points (round-to-nearest-even, what `astype(bfloat16)` does) and `bf16=False`
to run entirely in fp32, the form the tests pin against the transformers fp32
modules and brute-force closed forms.

Pinning status (see tests/test_oracle_*.py):
  attention  — brute-force per-(b,h,i) loops (window, padding, GQA, softcap),
               dense closed form, TF Gemma-2 eager attention (fp32).
  rmsnorm, gated MLP, RoPE — TF Gemma2RMSNorm / Gemma2MLP / rotary (fp32),
               RoPE invariants (position 0 fixed, norm preserved).
  decision forward + readout — TF Gemma2ForCausalLM logits (fp32, tiny
               config) read at the option positions and label ids.
  decode     — the reference's KATs (tests/clef/test_input.py:42-44, 78-83).
  bf16 rounding — bit patterns against torch.bfloat16 casts.
"""
