"""vLLM integration: decoder adapter, decode guard/route, backend registration.

``native_decode`` and ``decoder_adapter`` import without vLLM; ``vllm_plugin``
defines the vLLM backend classes and needs vLLM installed.
"""
