"""MI355X-native (gfx950) TurboQuant Pro KV cache: quantize-on-append and fused
decode-on-codes attention behind the reference's cache API.

The compute path is the HIP library ``lib/libtqk.so`` (C ABI in
``include/tqk.h``); this package is the host side that plans launches and
mirrors the reference interface.
"""

__version__ = "0.1.0"

from .codebooks import group_tokens_for, n_groups_for, random_rotation, value_codebook  # noqa: F401
from .pool import TQKVPool  # noqa: F401
from .core import TurboQuantKVCache, merge_partials  # noqa: F401
from .autoconfig import AutoConfig, list_models, list_targets  # noqa: F401
from .vllm_plugin import TurboQuantKVBackend, TurboQuantKVManager  # noqa: F401
from . import plugins  # noqa: F401
