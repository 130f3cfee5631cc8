"""``attnfuse.integrations.hf`` names the same module object as
``attentionfuse_amd.integrations.hf`` (one registration, one graph cache)."""
import sys

from attentionfuse_amd.integrations import hf as _hf

sys.modules[__name__] = _hf
