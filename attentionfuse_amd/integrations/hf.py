"""HuggingFace ``attn_implementation="attnfuse"`` backend.

Same registration, name and signature as the reference
(attnfuse/integrations/hf.py:56-66,127-145): importing this module puts
``attnfuse_attention_forward`` into transformers' ``ALL_ATTENTION_FUNCTIONS``
under "attnfuse", after which a model opts in with
``model.config._attn_implementation = "attnfuse"`` or
``attn_implementation="attnfuse"``.

The function keeps transformers' attention contract: ``query`` is
(B, H_q, N_q, D), ``key``/``value`` are (B, H_kv, N_kv, D) with RoPE already
applied by the model, and the return value is ``(attn_output, None)`` with
``attn_output`` laid out (B, N_q, H_q, D) contiguous, as the model's
``reshape`` after the call expects.  GQA is handled by the kernels (no
``repeat_kv``).  ``scaling`` is the softmax scale.

Routing (the fused path runs whenever the call is one of its cases):

* no dropout and either no mask or a mask equal to the plain causal pattern;
* causal with N_q == N_kv -> fused causal kernel; N_q == 1 -> flash
  decoding over the whole cache; non-causal -> dense kernel;
* anything else (dropout, padding / sliding-window / custom masks, causal
  chunks with N_q != N_kv, head sizes or dtypes without an instantiated
  kernel, CPU tensors) -> transformers' own SDPA function, so results equal
  ``attn_implementation="sdpa"``.

Where it deliberately differs from the reference: the output is returned in
transformers' (B, N, H, D) layout (the reference returns (B, H, N, D),
hf.py:99-102); ``scaling`` is honoured (the reference drops it); a mask is
accepted only if it equals the causal pattern element for element (the
reference looks at one corner element, hf.py:118-123); and a mask builder
is registered for "attnfuse" (transformers' SDPA builder), because for an
attention name without one transformers builds no mask at all, which would
drop padding information.
"""
from __future__ import annotations

import weakref
from typing import Optional, Tuple

import torch

import attentionfuse_amd as af

_GRAPH_CACHE: dict = {}
_MASK_CACHE: dict = {}


def _get_attn_fn(head_dim: int, dtype: torch.dtype, is_causal: bool,
                 scaling: Optional[float]):
    """The traced attention function for one (D, dtype, causal, scale) cell
    (reference hf.py:36-53, with the scale added to the key)."""
    key = (head_dim, str(dtype), is_causal, scaling)
    fn = _GRAPH_CACHE.get(key)
    if fn is not None:
        return fn
    if is_causal:
        @af.attention
        def attn(Q, K, V):
            return af.softmax(af.causal(af.scaled_dot_product(Q, K, scaling))) @ V
    else:
        @af.attention
        def attn(Q, K, V):
            return af.softmax(af.scaled_dot_product(Q, K, scaling)) @ V
    _GRAPH_CACHE[key] = attn
    return attn


def _is_pure_causal_mask(mask: Optional[torch.Tensor], n_q: int, n_kv: int) -> bool:
    """True iff ``mask`` allows exactly the keys j <= i for every query i of
    every batch entry: a bool mask (True = attend) or an additive mask
    (0 = attend, -inf or the dtype minimum = masked) of shape
    (B or 1, 1 or H, N_q, N_kv).  ``None`` counts as causal."""
    if mask is None:
        return True
    if mask.dim() != 4 or mask.shape[-2] != n_q or mask.shape[-1] != n_kv or n_q != n_kv:
        return False
    # transformers hands the same mask object to every layer of a forward:
    # remember the answer for that object (weakly, and for its current
    # contents) so the check runs once per forward
    ent = _MASK_CACHE.get(id(mask))
    if ent is not None and ent[0]() is mask and ent[1] == mask._version:
        return ent[2]
    ok = _causal_pattern(mask, n_q, n_kv)
    if len(_MASK_CACHE) > 64:
        _MASK_CACHE.clear()
    _MASK_CACHE[id(mask)] = (weakref.ref(mask), mask._version, ok)
    return ok


def _causal_pattern(mask: torch.Tensor, n_q: int, n_kv: int) -> bool:
    allowed = mask if mask.dtype == torch.bool else (mask == 0)
    if mask.dtype != torch.bool:
        blocked = torch.isinf(mask) | (mask <= torch.finfo(mask.dtype).min / 2)
        if not bool((allowed | blocked).all()):
            return False
    tri = torch.ones(n_q, n_kv, dtype=torch.bool, device=mask.device).tril()
    return bool((allowed == tri).all())


def _sdpa(module, query, key, value, attention_mask, dropout, scaling, is_causal, **kwargs):
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    return ALL_ATTENTION_FUNCTIONS["sdpa"](
        module, query, key, value, attention_mask,
        dropout=dropout, scaling=scaling, is_causal=is_causal, **kwargs)


def plan(module, query, key, attention_mask, dropout, is_causal) -> str:
    """'causal', 'dense' (incl. decode) or 'sdpa' for this call (device
    aside: the caller sends non-GPU tensors to SDPA)."""
    if dropout > 0.0:
        return "sdpa"
    if is_causal is None:
        is_causal = getattr(module, "is_causal", True)
    n_q, n_kv = query.shape[2], key.shape[2]
    causal = bool(is_causal) and n_q > 1
    if attention_mask is not None:
        if not (causal and _is_pure_causal_mask(attention_mask, n_q, n_kv)):
            return "sdpa"
    if causal and n_q != n_kv:
        return "sdpa"
    return "causal" if causal else "dense"


def attnfuse_attention_forward(
    module: torch.nn.Module,
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    attention_mask: Optional[torch.Tensor],
    dropout: float = 0.0,
    scaling: Optional[float] = None,
    is_causal: Optional[bool] = None,
    **kwargs,
) -> Tuple[torch.Tensor, None]:
    """AttnFuse drop-in for transformers' attention interface (reference
    hf.py:56-102); see the module docstring for the routing."""
    route = plan(module, query, key, attention_mask, dropout, is_causal)
    if route == "sdpa" or query.device.type != "cuda":
        return _sdpa(module, query, key, value, attention_mask, dropout, scaling,
                     is_causal, **kwargs)
    from ..runtime.kernel_cache import get_or_compile
    fn = _get_attn_fn(query.shape[-1], query.dtype, route == "causal", scaling)
    try:
        get_or_compile(fn(query, key, value, return_graph=True))
    except NotImplementedError:
        return _sdpa(module, query, key, value, attention_mask, dropout, scaling,
                     is_causal, **kwargs)
    B, H, n_q, D = query.shape
    if torch.is_grad_enabled() and any(t.requires_grad for t in (query, key, value)):
        return fn(query, key, value).transpose(1, 2).contiguous(), None
    # the kernel writes straight into the (B, N, H, D) buffer through a
    # (B, H, N, D) view of it
    out = torch.empty(B, n_q, H, D, dtype=query.dtype, device=query.device)
    fn(query, key, value, out=out.transpose(1, 2))
    return out, None


def register():
    """Register the ``attnfuse`` attention function and its mask builder
    with transformers (reference hf.py:127-141).  Safe to call repeatedly."""
    try:
        from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS, sdpa_mask
        from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    except ImportError as e:  # pragma: no cover
        raise ImportError("transformers >= 4.40 is required for the AttnFuse "
                          "integration") from e
    ALL_ATTENTION_FUNCTIONS.register("attnfuse", attnfuse_attention_forward)
    ALL_MASK_ATTENTION_FUNCTIONS.register("attnfuse", sdpa_mask)


register()
