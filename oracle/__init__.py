"""CPU oracle of the verify hot path -- TEST INFRASTRUCTURE, not product code.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and only as what the
HIP results are compared against (or, for the CPU baseline, as the thing timed on the host cores). The product
path (nvs_amd) never imports it and has no CPU fallback.

Modules
  oracle.attention     paged KV store and paged multi-query attention: an fp64 numpy brute force and a torch fp32
                       restatement of the reference's CPU stand-in (tests/fake_paged_attention.py)
  oracle.spec_sampler  torch-CPU restatement of nanovllm/layers/spec_sampler.py, with the random draws passed in
  oracle.qk_norm_rope  eager q/k RMSNorm + rotary embedding + KV store (layernorm.py, rotary_embedding.py, qwen3.py)
  oracle.layernorm     the decoder layer's RMSNorm (with the residual add) and SiLU-and-mul (layernorm.py,
                       activation.py)
  oracle.markov        DSpark's Markov rows with candidate rows (speculative.py:145-184)

How each function is pinned (each check fails for a dropped term, a wrong sign or index, a transposed operand):
  attention.store_kvcache       exact-copy semantics, a known slot layout (tests/test_oracle_attention.py)
  attention.paged_attention_f64 closed forms (one visible key -> that V row; equal keys -> mean of visible V;
                                scale 0 -> mean), a dense-attention brute force with an explicit mask, GQA head
                                mapping by construction, block-table permutation invariance
  attention.paged_attention_t32 agreement with the fp64 brute force (fp32 tolerance)
  qk_norm_rope.*                RMSNorm closed forms and fp64, the rotary table against its frequency formula, the
                                rotation against the fp64 complex product (identity at 0, composition, norms,
                                relative-position scores), a planted interleaved rotation that must differ
  layernorm.*                   a constant row normalising to the weight, a known vector with and without eps, the
                                fp64 mathematics, the residual semantics (rounded sum out, norm of the unrounded
                                sum), SiLU closed forms and a swapped gate/up half that must differ
  markov.*                      the four known answers of the reference's tests/test_dspark_propose.py, a forcing
                                bias only the previous row's token can follow, one kept token winning whatever the
                                noise
  spec_sampler.*                every known answer of the reference's tests/test_spec_sampler.py, the
                                fixed-length body the variable-length rewrite must reproduce bit for bit, exact
                                Fraction enumeration of the frozen cases (SHA-256 pinned), Hoeffding-bound
                                output distributions of whole speculative rounds
No function here is left "parity unpinned".
"""
