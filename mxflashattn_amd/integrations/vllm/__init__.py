"""vLLM integration: decoder adapter, decode guard/route, backend registration.

``native_decode``, ``decoder_adapter`` and ``compat`` (the vLLM release gate)
import without vLLM; ``vllm_plugin`` defines the vLLM backend classes and needs
vLLM installed.
"""
