"""nanokv-llm_amd: the attention hot path of nano-kvllm on MI355X (gfx950).

Host side in Python on PyTorch-ROCm; all compute in libnkv_amd.so
(hand-written HIP kernels behind the C ABI of include/nkv.h). The package
directory name is not a Python identifier; import it with
``importlib.import_module("nanokv-llm_amd")``.
"""
from .layers.attention import (Attention, paged_decode, release_retired_decode_workspaces,
                               reserve_decode_workspace, store_kvcache, varlen_prefill)
from .layers.compress_utils import MyCompressCompact
from .layers.CompressMethod import SnapKV
from .layers.rotary_embedding import RotaryEmbedding, get_rope, qk_norm_rope_store
from .utils.context import Context, get_context, set_context, reset_context

__all__ = [
    "Attention", "store_kvcache", "paged_decode", "reserve_decode_workspace",
    "release_retired_decode_workspaces", "varlen_prefill",
    "MyCompressCompact",
    "SnapKV", "Context", "get_context", "set_context", "reset_context", "RotaryEmbedding",
    "get_rope", "qk_norm_rope_store",
]
