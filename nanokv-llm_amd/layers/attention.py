"""Drop-in Attention layer and the functional ops behind it.

Mirrors nanokvllm/layers/attention.py: ``store_kvcache`` (:33-40) and
``Attention`` (:42-108) with the same constructor, attributes
(``k_cache``/``v_cache`` assigned by the model runner) and ``forward(q, k, v,
Layer)``. Every op runs in libnkv_amd.so on the caller's current HIP stream;
nothing here computes on the CPU.
"""
from __future__ import annotations

import torch
from torch import nn

from .. import _lib
from ..utils.context import get_context
from .compress_utils import MyCompressCompact

_BF16 = torch.bfloat16


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, slot_mapping: torch.Tensor, k_scale: float = 1.0,
                  v_scale: float = 1.0) -> None:
    """k_cache/v_cache row slot_mapping[i] <- key[i]/value[i]; -1 slots skipped.

    Same checks as the reference (attention.py:33-40): last dim contiguous,
    head stride == head_dim, cache token stride == Hk*D, one slot per token.
    bf16 or fp16 rows go to a cache of the same dtype (the copy moves 2-byte
    elements); an fp8 (float8_e4m3fn) cache stores E4M3FN(clamp(x / scale)) of
    bf16 rows.
    """
    N, num_heads, head_dim = key.shape
    D = num_heads * head_dim
    _lib.require_device(key.device, value=value, k_cache=k_cache, v_cache=v_cache,
                        slot_mapping=slot_mapping)
    _lib.need(value.shape == key.shape, "store_kvcache: value shape differs from key")
    _lib.need(v_cache.shape == k_cache.shape and v_cache.dtype == k_cache.dtype,
              "store_kvcache: v_cache shape/dtype differ from k_cache")
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert key.stride(1) == head_dim and value.stride(1) == head_dim
    assert k_cache.stride(1) == D and v_cache.stride(1) == D
    assert slot_mapping.numel() == N
    assert slot_mapping.dtype == torch.int32 and slot_mapping.is_contiguous()
    n_slots = k_cache.numel() // D
    if k_cache.dtype == torch.float8_e4m3fn:
        assert v_cache.dtype == k_cache.dtype and key.dtype == _BF16 and value.dtype == _BF16
        rc = _lib.lib().nkv_store_kvcache_fp8(
            key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0),
            k_cache.data_ptr(), v_cache.data_ptr(), slot_mapping.data_ptr(), N, num_heads,
            head_dim, n_slots, float(k_scale), float(v_scale), _lib.stream_of(key))
        _lib.check(rc, "store_kvcache_fp8")
        return
    _lib.is_f16(key, "store_kvcache: key")
    _lib.need(value.dtype == key.dtype and k_cache.dtype == key.dtype,
              "store_kvcache: key, value and the caches must share one dtype")
    rc = _lib.lib().nkv_store_kvcache(
        key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0),
        k_cache.data_ptr(), v_cache.data_ptr(), slot_mapping.data_ptr(), N,
        num_heads, head_dim, n_slots, _lib.stream_of(key))
    _lib.check(rc, "store_kvcache")


def _decode_args(q, k_cache, block_tables, context_lens, v_cache=None, out=None):
    _lib.require_device(q.device, k_cache=k_cache, v_cache=v_cache, block_tables=block_tables,
                        context_lens=context_lens, out=out)
    bs, Hq, D = q.shape
    NB, B, Hk, Dk = k_cache.shape
    _lib.is_f16(q, "paged_decode: q")
    _lib.need(k_cache.dtype == q.dtype or (k_cache.dtype == torch.float8_e4m3fn
                                           and q.dtype == _BF16),
              "paged_decode: caches must have q's dtype (or fp8 with bf16 q)")
    if v_cache is not None:
        _lib.need(v_cache.shape == k_cache.shape and v_cache.dtype == k_cache.dtype
                  and v_cache.is_contiguous(),
                  "paged_decode: v_cache must be contiguous with k_cache's shape and dtype")
    if out is not None:
        _lib.need(out.shape == q.shape and out.dtype == q.dtype and out.stride(-1) == 1
                  and out.stride(1) == D, "paged_decode: out must be [bs, Hq, D] in q's dtype, "
                  "rows of contiguous heads")
    assert Dk == D and q.stride(-1) == 1 and q.stride(1) == D
    assert k_cache.is_contiguous()
    assert block_tables.dtype == torch.int32 and block_tables.stride(1) == 1
    assert context_lens.dtype == torch.int32 and context_lens.is_contiguous()
    assert block_tables.size(0) >= bs and context_lens.numel() >= bs
    return bs, Hq, D, NB, B, Hk


def decode_workspace_bytes(bs: int, n_q_heads: int, max_blocks_per_seq: int,
                           block_size: int, head_dim: int = 128) -> int:
    """Bytes nkv_paged_decode needs: partial rows for what the grid can write (resident
    waves x 16 query heads + batch x Hq rows of 528 B), not batch x table width."""
    return int(_lib.lib().nkv_paged_decode_workspace_bytes(bs, n_q_heads, head_dim,
                                                            max_blocks_per_seq, block_size))


def paged_decode_workspace(q: torch.Tensor, k_cache: torch.Tensor,
                           block_tables: torch.Tensor) -> torch.Tensor:
    bs, Hq, D = q.shape
    nbytes = decode_workspace_bytes(bs, Hq, block_tables.size(1), k_cache.size(1), D)
    return torch.empty(max(nbytes, 4), dtype=torch.uint8, device=q.device)


# One decode workspace per device, shared by every Attention layer: the layers of a step
# run one after another on one stream, so no two decode calls use it at once (callers
# that run layers concurrently on several streams pass their own workspaces to
# paged_decode). It only grows. A replaced buffer that a HIP graph captured (a decode call
# ran during capture while it was current) is kept alive, because that graph still holds
# its address; one that no capture saw is freed. release_retired_decode_workspaces() drops
# the kept ones once the caller has dropped its graphs.
_SHARED_WS: dict = {}
_CAPTURED_WS: set = set()  # (device, data_ptr) of shared workspaces seen during a capture
_RETIRED_WS: list = []


def shared_decode_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """The device's shared decode workspace, grown to at least ``nbytes``."""
    ws = _SHARED_WS.get(device)
    capturing = torch.cuda.is_current_stream_capturing()
    if ws is None or ws.numel() < nbytes:
        if capturing:
            raise _lib.NkvError(
                "the shared decode workspace must be large enough before graph capture: "
                "call reserve_decode_workspace (or run the largest batch eagerly) first")
        size = max(int(nbytes), 4)
        if ws is not None:
            size = max(size, 2 * ws.numel())  # few regrowths
            key = (device, ws.data_ptr())
            if key in _CAPTURED_WS:  # a captured graph may still read and write it
                _CAPTURED_WS.discard(key)
                _RETIRED_WS.append(ws)
        ws = torch.empty(size, dtype=torch.uint8, device=device)
        _SHARED_WS[device] = ws
    if capturing:
        _CAPTURED_WS.add((device, ws.data_ptr()))
    return ws


def release_retired_decode_workspaces() -> int:
    """Free the replaced shared workspaces that graphs captured; call after dropping every
    graph captured before the last regrowth. Returns how many were released."""
    n = len(_RETIRED_WS)
    _RETIRED_WS.clear()
    return n


def reserve_decode_workspace(device, max_num_seqs: int, n_q_heads: int,
                             max_blocks_per_seq: int, block_size: int,
                             head_dim: int = 128) -> torch.Tensor:
    """Size the device's shared decode workspace for the largest decode batch (the
    model runner's max_num_seqs / graph batch and table width), e.g. before capture."""
    device = torch.device(device)
    if device.type == "cuda" and device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    return shared_decode_workspace(device, decode_workspace_bytes(
        max_num_seqs, n_q_heads, max_blocks_per_seq, block_size, head_dim))


def paged_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                 context_lens: torch.Tensor, block_tables: torch.Tensor, scale: float,
                 out: torch.Tensor | None = None,
                 workspace: torch.Tensor | None = None, k_scale: float = 1.0,
                 v_scale: float = 1.0) -> torch.Tensor:
    """Paged GQA decode: q [bs, Hq, D] -> out [bs, Hq, D] (q's dtype: bf16 or fp16).

    Same math as flash_attn_with_kvcache(q.unsqueeze(1), k_cache, v_cache,
    cache_seqlens=context_lens, block_table=block_tables, softmax_scale=scale,
    causal=True) at attention.py:104-107. fp8 (float8_e4m3fn) caches are read
    as code * k_scale / code * v_scale.
    """
    bs, Hq, D, NB, B, Hk = _decode_args(q, k_cache, block_tables, context_lens, v_cache, out)
    if out is None:
        out = torch.empty(bs, Hq, D, dtype=q.dtype, device=q.device)
    if workspace is None:
        workspace = paged_decode_workspace(q, k_cache, block_tables)
    if k_cache.dtype == torch.float8_e4m3fn:
        assert v_cache.dtype == k_cache.dtype and v_cache.is_contiguous()
        rc = _lib.lib().nkv_paged_decode_fp8(
            q.data_ptr(), q.stride(0), k_cache.data_ptr(), v_cache.data_ptr(),
            block_tables.data_ptr(), block_tables.stride(0), context_lens.data_ptr(), bs, Hq,
            Hk, D, B, block_tables.size(1), NB, float(scale), float(k_scale), float(v_scale),
            out.data_ptr(), out.stride(0), workspace.data_ptr(), workspace.numel(),
            _lib.stream_of(q))
        _lib.check(rc, "paged_decode_fp8")
        return out
    fn = _lib.lib().nkv_paged_decode_f16 if q.dtype == torch.float16 else \
        _lib.lib().nkv_paged_decode
    rc = fn(q.data_ptr(), q.stride(0), k_cache.data_ptr(), v_cache.data_ptr(),
            block_tables.data_ptr(), block_tables.stride(0), context_lens.data_ptr(), bs, Hq, Hk,
            D, B, block_tables.size(1), NB, float(scale), out.data_ptr(), out.stride(0),
            workspace.data_ptr(), workspace.numel(), _lib.stream_of(q))
    _lib.check(rc, "paged_decode")
    return out


def varlen_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                   cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor, max_seqlen_q: int,
                   scale: float, block_tables: torch.Tensor | None = None,
                   out: torch.Tensor | None = None, max_seqlen_k: int | None = None,
                   k_scale: float = 1.0, v_scale: float = 1.0) -> torch.Tensor:
    """Varlen causal (bottom-right) attention: q [sum Lq, Hq, D] -> [sum Lq, Hq, D].

    With ``block_tables`` k/v are the paged caches [NB, B, Hk, D]; without,
    they are [sum Lk, Hk, D] rows, each with its own row stride (k roped and
    contiguous, v a view of the qkv projection). Same math as
    flash_attn_varlen_func(..., causal=True, block_table) at attention.py:96-102.
    q, k, v and the output are bf16 or fp16 (one dtype); an fp8 pool takes bf16 q.
    """
    N, Hq, D = q.shape
    _lib.require_device(q.device, k=k, v=v, cu_seqlens_q=cu_seqlens_q, cu_seqlens_k=cu_seqlens_k,
                        block_tables=block_tables, out=out)
    assert q.stride(-1) == 1 and q.stride(1) == D
    assert cu_seqlens_q.dtype == torch.int32 and cu_seqlens_k.dtype == torch.int32
    n_seqs = cu_seqlens_q.numel() - 1
    f16 = _lib.is_f16(q, "varlen_prefill: q")
    _lib.need(cu_seqlens_k.numel() == n_seqs + 1 and cu_seqlens_q.is_contiguous()
              and cu_seqlens_k.is_contiguous(),
              "varlen_prefill: cu_seqlens_q/k must be contiguous, one entry per sequence + 1")
    _lib.need(v.dtype == k.dtype, "varlen_prefill: k and v dtypes differ")
    if out is not None:
        _lib.need(out.shape == q.shape and out.dtype == q.dtype and out.stride(-1) == 1
                  and out.stride(1) == D, "varlen_prefill: out must be shaped like q, in q's "
                  "dtype, rows of contiguous heads")
    if block_tables is not None and k.dtype == torch.float8_e4m3fn:
        # fp8 pool: the kernel widens the codes as it stages them (no bf16 copy)
        NB, B, Hk, Dk = k.shape
        _lib.need(not f16, "varlen_prefill: an fp8 pool is read with bf16 q")
        _lib.need(v.shape == k.shape and k.is_contiguous() and v.is_contiguous(),
                  "varlen_prefill: fp8 caches must be contiguous, v shaped like k")
        _lib.need(block_tables.dtype == torch.int32 and block_tables.stride(1) == 1,
                  "varlen_prefill: block_tables must be int32 rows")
        assert Dk == D
        if out is None:
            out = torch.empty(N, Hq, D, dtype=_BF16, device=q.device)
        rc = _lib.lib().nkv_prefill_varlen_fp8(
            q.data_ptr(), q.stride(0), k.data_ptr(), v.data_ptr(), cu_seqlens_q.data_ptr(),
            cu_seqlens_k.data_ptr(), block_tables.data_ptr(), block_tables.stride(0),
            block_tables.size(1), n_seqs, int(max_seqlen_q), Hq, Hk, D, B, NB, float(scale),
            float(k_scale), float(v_scale), out.data_ptr(), out.stride(0), _lib.stream_of(q))
        _lib.check(rc, "varlen_prefill_fp8")
        return out
    if block_tables is not None:
        NB, B, Hk, Dk = k.shape
        assert k.is_contiguous() and v.is_contiguous() and v.shape == k.shape
        _lib.need(k.dtype == q.dtype, "varlen_prefill: paged caches must have q's dtype "
                  "(or be fp8)")
        k_row_stride = v_row_stride = Hk * Dk
        n_rows = NB * B
        bt_ptr, bt_stride = block_tables.data_ptr(), block_tables.stride(0)
        max_blocks = block_tables.size(1)
        assert block_tables.dtype == torch.int32 and block_tables.stride(1) == 1
    else:
        _, Hk, Dk = k.shape
        assert v.shape == k.shape
        _lib.need(k.dtype == q.dtype, "varlen_prefill: contiguous k/v must have q's dtype")
        assert k.stride(1) == Dk and k.stride(2) == 1 and v.stride(1) == Dk and v.stride(2) == 1
        k_row_stride, v_row_stride = k.stride(0), v.stride(0)
        n_rows = k.size(0)
        B = 0
        bt_ptr, bt_stride, max_blocks = None, 0, 0
    assert Dk == D
    if out is None:
        out = torch.empty(N, Hq, D, dtype=q.dtype, device=q.device)
    fn = _lib.lib().nkv_prefill_varlen_f16 if f16 else _lib.lib().nkv_prefill_varlen
    rc = fn(
        q.data_ptr(), q.stride(0), k.data_ptr(), v.data_ptr(), k_row_stride, v_row_stride,
        cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr(), bt_ptr, bt_stride, max_blocks, n_seqs,
        int(max_seqlen_q), Hq, Hk, D, B, n_rows, float(scale), out.data_ptr(), out.stride(0),
        _lib.stream_of(q))
    _lib.check(rc, "varlen_prefill")
    return out


class Attention(nn.Module):
    """Per-layer attention: store -> (periodic compression) -> prefill or decode.

    Constructor and forward follow nanokvllm/layers/attention.py:44-108.
    """

    def __init__(self, num_heads, head_dim, scale, num_kv_heads, vllm_config, num_layers):
        super().__init__()
        # the kernels' limits, checked here rather than at the first forward or the first
        # compression step mid-serving (include/nkv.h states each of them)
        _lib.need(head_dim in (64, 128, 256), f"Attention: head_dim {head_dim} is not 64, "
                  "128 or 256")
        _lib.need(num_kv_heads > 0 and num_heads % num_kv_heads == 0,
                  f"Attention: num_heads {num_heads} is not a multiple of num_kv_heads "
                  f"{num_kv_heads}")
        max_group = 64 if head_dim == 256 else 128  # prefill: every tile holds a query per head
        _lib.need(num_heads // num_kv_heads <= max_group,
                  f"Attention: GQA group {num_heads // num_kv_heads} above {max_group}")
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.k_cache = self.v_cache = torch.tensor([])
        self.k_scale = self.v_scale = 1.0  # fp8 pools (KVCachePool.bind sets them)

        self.kv_compress_enabled = vllm_config.kv_compress_enabled
        if self.kv_compress_enabled:
            self.num_layers = num_layers
            self.kv_compress_window_blocks = vllm_config.kv_compress_window_blocks
            self.kv_compress_keep_blocks = vllm_config.kv_compress_keep_blocks
            self.kv_compress_keep_extra_tokens = vllm_config.kv_compress_keep_extra_tokens
            self.kv_compress_agg = getattr(vllm_config, "kv_compress_agg", "all")
            W = self.kv_compress_window_blocks
            _lib.need(0 < W <= 64, f"Attention: kv_compress_window_blocks {W} not in 1..64")
            _lib.need(self.kv_compress_keep_blocks >= 0 and
                      self.kv_compress_keep_extra_tokens >= 0,
                      "Attention: kv_compress_keep_blocks and kv_compress_keep_extra_tokens "
                      "must be >= 0")
            _lib.need(self.kv_compress_agg in ("all", "group"),
                      f"Attention: kv_compress_agg {self.kv_compress_agg!r} is not 'all' or "
                      "'group'")
        self._cache_checked = None  # (k_cache data_ptr, shape) whose geometry was checked

    def _check_cache(self):
        """The bound cache's geometry against the kernels' limits, once per binding: block
        size a multiple of 16 (decode, prefill); with compression, a window of at most 4096
        candidates (W*B - 1) and a block size the compression kernels take (a multiple of 64
        with W*B <= 1024, or of 256)."""
        kc = self.k_cache
        key = (kc.data_ptr(), tuple(kc.shape))
        if self._cache_checked == key:
            return
        _lib.need(kc.dim() == 4 and kc.size(2) == self.num_kv_heads and
                  kc.size(3) == self.head_dim,
                  f"Attention: k_cache must be [blocks, block_size, {self.num_kv_heads}, "
                  f"{self.head_dim}], got {tuple(kc.shape)}")
        B = kc.size(1)
        _lib.need(B % 16 == 0, f"Attention: block_size {B} is not a multiple of 16")
        if self.kv_compress_enabled:
            Lw = self.kv_compress_window_blocks * B
            keep = self.kv_compress_keep_blocks * B + self.kv_compress_keep_extra_tokens
            _lib.need(Lw - 1 <= 4096, f"Attention: compression window of {Lw} tokens above "
                      "4097")
            _lib.need((B % 64 == 0 and Lw <= 1024) or B % 256 == 0,
                      f"Attention: compression needs block_size a multiple of 64 (window <= "
                      f"1024 tokens) or of 256, got {B}")
            # keep >= Lw is the reference's no-op (SnapKV returns False, CompressMethod.py:17-18)
            _lib.need(keep > 2, f"Attention: {keep} kept tokens (bos, selected, latest: > 2)")
        self._cache_checked = key

    def _workspace(self, q, block_tables):
        """The device's decode workspace, shared with every other layer."""
        return shared_decode_workspace(q.device, decode_workspace_bytes(
            q.size(0), q.size(1), block_tables.size(1), self.k_cache.size(1), q.size(2)))

    def forward(self, q: torch.Tensor, k: torch.Tensor | None, v: torch.Tensor, Layer,
                kv_stored: bool = False):
        """``kv_stored=True``: k/v were already written to the cache (by
        qk_norm_rope_store); k may then be None unless prefill reads it
        contiguously (no block table)."""
        context = get_context()
        k_cache, v_cache = self.k_cache, self.v_cache
        if k_cache.numel():
            self._check_cache()
        if k_cache.numel() and v_cache.numel() and not kv_stored:
            store_kvcache(k, v, k_cache, v_cache, context.slot_mapping, self.k_scale,
                          self.v_scale)

        if (context.use_decode_kernel and self.kv_compress_enabled and context.is_compress_step
                and (context.compress_selected_batch_indices
                     or context.compress_seq_idx is not None)):
            MyCompressCompact(
                q_current=q, k_cache=k_cache, v_cache=v_cache, layer_id=Layer,
                block_size=k_cache.size(1), window_blocks=self.kv_compress_window_blocks,
                keep_blocks=self.kv_compress_keep_blocks,
                keep_extra_tokens=self.kv_compress_keep_extra_tokens,
                num_layers=self.num_layers, context=context, agg=self.kv_compress_agg,
                k_scale=self.k_scale)

        if not context.use_decode_kernel:
            if context.block_tables is not None:  # K/V read back from the paged cache
                return varlen_prefill(q, k_cache, v_cache, context.cu_seqlens_q,
                                      context.cu_seqlens_k, context.max_seqlen_q, self.scale,
                                      block_tables=context.block_tables,
                                      max_seqlen_k=context.max_seqlen_k, k_scale=self.k_scale,
                                      v_scale=self.v_scale)
            return varlen_prefill(q, k, v, context.cu_seqlens_q, context.cu_seqlens_k,
                                  context.max_seqlen_q, self.scale)
        o = paged_decode(q, k_cache, v_cache, context.context_lens, context.block_tables,
                         self.scale, workspace=self._workspace(q, context.block_tables),
                         k_scale=self.k_scale, v_scale=self.v_scale)
        return o.unsqueeze(1)
