from .configuration_llama_seerattn import SeerAttnLlamaConfig
from .modeling_llama_flashprefill_compactattn import (LlamaFlashPrefillCompactAttnAttention,
                                                      SeerAttnLlamaFlashPrefillCompactAttnForCausalLM)
from .modeling_llama_seerattn_chunked_dense import LlamaSeerAttentionChunkedDense, SeerAttnLlamaChunkedDenseForCausalLM

__all__ = [
    "SeerAttnLlamaConfig",
    "LlamaSeerAttentionChunkedDense",
    "SeerAttnLlamaChunkedDenseForCausalLM",
    "LlamaFlashPrefillCompactAttnAttention",
    "SeerAttnLlamaFlashPrefillCompactAttnForCausalLM",
]
