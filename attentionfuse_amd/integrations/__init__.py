"""Integrations with downstream libraries (reference
attnfuse/integrations/__init__.py).

``import attentionfuse_amd.integrations.hf`` (or ``attnfuse.integrations.hf``)
registers the "attnfuse" attention implementation with HuggingFace
transformers, so a Llama-class model runs its attention on the fused
kernels with ``model.config._attn_implementation = "attnfuse"``.
"""
