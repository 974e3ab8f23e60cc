from naivllm_amd.layers.attention import Attention, paged_attention_verify, store_kvcache

__all__ = ["Attention", "paged_attention_verify", "store_kvcache"]
