"""Per-step attention metadata shared by every Attention layer.

Same fields, defaults and functions as nanokvllm/utils/context.py:3-40, so a
model runner written for the reference fills it unchanged; two more fields
carry the device-side compression selection and its events.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class Context:
    use_decode_kernel: bool = False
    cu_seqlens_q: torch.Tensor | None = None
    cu_seqlens_k: torch.Tensor | None = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: torch.Tensor | None = None
    context_lens: torch.Tensor | None = None
    block_tables: torch.Tensor | None = None

    compression_events: list | None = None
    compress_need_mask: list | None = None
    compress_any: bool = False

    is_compress_step: bool = False
    compress_selected_batch_indices: list | None = None
    compress_selected_seq_ids: list[int] | None = None
    compress_base_context_lens: torch.Tensor | None = None

    # device-side selection (graph-capturable compression step): int32 [topk], -1 padded,
    # filled on the device by nkv_compress_schedule; the last layer then leaves its event
    # rows in compression_events_device for the host to apply after the step
    compress_seq_idx: torch.Tensor | None = None
    compression_events_device: torch.Tensor | None = None


_CONTEXT = Context()


def get_context() -> Context:
    return _CONTEXT


def set_context(use_decode_kernel, cu_seqlens_q=None, cu_seqlens_k=None, max_seqlen_q=0,
                max_seqlen_k=0, slot_mapping=None, context_lens=None, block_tables=None):
    """Install a fresh Context (context.py:27-36): compression fields reset."""
    global _CONTEXT
    _CONTEXT = Context(use_decode_kernel, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                       slot_mapping, context_lens, block_tables,
                       compression_events=[],
                       compress_need_mask=None,
                       compress_any=False,
                       is_compress_step=False,
                       compress_selected_batch_indices=None,
                       compress_selected_seq_ids=None,
                       compress_base_context_lens=None)


def reset_context():
    global _CONTEXT
    _CONTEXT = Context()
