"""Runtime: launch bundles, dispatch and the C-ABI binding."""
from .dispatch import run_attention
from .kernel_cache import clear_cache, get_or_compile

__all__ = ["run_attention", "get_or_compile", "clear_cache"]
