"""MI355X (gfx950) target-verify hot path of nano-vllm-speculative-decoding.

Drop-in replacements, same Python signatures as the reference:
  nvs_amd.layers.attention     Attention (verify / decode branches of Attention.forward), store_kvcache
  nvs_amd.layers.spec_sampler  probs_from_logits, truncate_logits, race, sample, accept_random(_varlen),
                               accept_greedy(_varlen) and the fused accept_from_logits
  nvs_amd.utils.context        Context / set_context / get_context / reset_context
Every op runs a hand-written HIP kernel from libnvs_amd.so through its C ABI (include/nvs_amd.h); there is no
fallback path: a missing library or a CPU tensor raises.
"""
__version__ = "0.1.0"
ABI_VERSION = 9
