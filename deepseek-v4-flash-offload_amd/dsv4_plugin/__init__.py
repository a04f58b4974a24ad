"""dsv4_plugin - DeepSeek-V4 routed-expert offload on MI355X (vLLM general plugin).

Entry point ``register_model`` (``vllm.general_plugins: dsv4_offload =
"dsv4_plugin:register_model"``) installs the MoE class swap and the expert
capture around ``load_weights``; idempotent, a no-op when no DeepSeek-V4 vLLM
model module is importable.
"""

from dsv4_plugin.models.deepseek_v4 import install_patches

__all__ = ["register_model"]


def register_model():
    install_patches()
