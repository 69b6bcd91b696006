"""Window-based periodic KV compression, run per layer inside Attention.forward.

Drop-in for ``MyCompressCompact`` (nanokvllm/layers/compress_utils.py:100-290):
same arguments, same return value, same side effects -- the layer's K/V cache
is compacted in place, ``context.context_lens`` of the selected sequences is
set to ``len - W*B + keep_tokens`` (from the base lengths captured before the
first layer), and on the last layer one event dict per selected sequence is
appended to ``context.compression_events``.

The reference's helpers ``get_tail_window_and_tail_slots`` and
``gather_kv_by_slots`` (:9-97) have no counterpart: window location is done
inside the kernels, and K is scored in place instead of being gathered.
Kernels (libnkv_amd.so): nkv_compress_step (scoring, importance, top-k and
compaction: one launch for agg "group", two for agg "all") on every layer,
nkv_compress_finalize on the last layer. nkv_compress_select and
nkv_compress_compact are the same work as separate calls.
"""
from __future__ import annotations

import torch

from .. import _lib

AGG_MODES = {"all": _lib.NKV_AGG_ALL, "group": _lib.NKV_AGG_GROUP}


class _StepBuffers:
    """Device buffers of one compression step, shared by all layers. ``selected`` is the
    host list of batch indices, or a device int32 tensor (-1 padded) selected on the
    device; then no host data enters the step and it can be captured in a HIP graph."""

    def __init__(self, selected, device, m, n_sets, n_cand, keep_tokens, ws_bytes, ev_len):
        self.key = _key(selected, device, n_sets, n_cand, keep_tokens, ws_bytes, ev_len)
        if torch.is_tensor(selected):
            self.seq_idx = selected
        else:
            self.seq_idx = torch.tensor(selected, dtype=torch.int32).to(device, non_blocking=True)
        self.importance = torch.empty(m, n_sets, n_cand, dtype=torch.float32, device=device)
        self.keep_idx = torch.empty(m, n_sets, keep_tokens, dtype=torch.int32, device=device)
        self.workspace = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=device)
        self.events = torch.empty(m, ev_len, dtype=torch.int32, device=device)


def _key(selected, device, n_sets, n_cand, keep_tokens, ws_bytes, ev_len):
    sel = ("device", selected.data_ptr(), selected.numel()) if torch.is_tensor(selected) \
        else tuple(selected)
    return (sel, device, n_sets, n_cand, keep_tokens, ws_bytes, ev_len)


def _buffers(context, selected, device, m, n_sets, n_cand, keep_tokens, ws_bytes, ev_len):
    key = _key(selected, device, n_sets, n_cand, keep_tokens, ws_bytes, ev_len)
    buf = getattr(context, "_nkv_compress_buffers", None)
    if buf is None or buf.key != key:
        buf = _StepBuffers(selected, device, m, n_sets, n_cand, keep_tokens, ws_bytes, ev_len)
        context._nkv_compress_buffers = buf
    return buf


def _check_window_args(what, q, k_cache, v_cache, block_tables, base_context_lens,
                       context_lens, seq_idx, importance, keep_idx, workspace, n_sets, n_cand,
                       keep_cols):
    """Device, dtype and shape checks shared by the compression wrappers: the library
    takes raw pointers and the geometry of k_cache, so every other tensor must agree."""
    _lib.require_device(k_cache.device, q=q, v_cache=v_cache, block_tables=block_tables,
                        base_context_lens=base_context_lens, context_lens=context_lens,
                        seq_idx=seq_idx, importance=importance, keep_idx=keep_idx,
                        workspace=workspace)
    for name, t in (("block_tables", block_tables), ("base_context_lens", base_context_lens),
                    ("context_lens", context_lens), ("seq_idx", seq_idx),
                    ("keep_idx", keep_idx)):
        if t is not None:
            _lib.need(t.dtype == torch.int32, f"{what}: {name} must be int32")
    _lib.need(block_tables.stride(1) == 1 and seq_idx.is_contiguous()
              and base_context_lens.is_contiguous(),
              f"{what}: block table rows, seq_idx and base_context_lens must be contiguous")
    _lib.need(context_lens is None or context_lens.is_contiguous(),
              f"{what}: context_lens must be contiguous")
    if v_cache is not None:
        _lib.need(v_cache.shape == k_cache.shape and v_cache.dtype == k_cache.dtype,
                  f"{what}: v_cache shape/dtype differ from k_cache")
    _lib.need(k_cache.is_contiguous() and (v_cache is None or v_cache.is_contiguous()),
              f"{what}: caches must be contiguous")
    if q is not None:
        D = k_cache.size(-1)
        _lib.is_f16(q, f"{what}: q")
        _lib.need(q.stride(-1) == 1 and q.stride(1) == D,
                  f"{what}: q must be rows of contiguous heads")
        _lib.need(k_cache.dtype == q.dtype or (k_cache.dtype == torch.float8_e4m3fn
                                               and q.dtype == torch.bfloat16),
                  f"{what}: the caches must have q's dtype (or be fp8 with bf16 q)")
    m = seq_idx.numel()
    if importance is not None:
        _lib.need(importance.dtype == torch.float32 and importance.is_contiguous()
                  and importance.shape == (m, n_sets, n_cand),
                  f"{what}: importance must be contiguous fp32 [{m}, {n_sets}, {n_cand}]")
    if keep_idx is not None and keep_cols is not None:
        _lib.need(keep_idx.is_contiguous() and keep_idx.shape == (m, n_sets, keep_cols),
                  f"{what}: keep_idx must be contiguous int32 [{m}, {n_sets}, {keep_cols}]")
    if workspace is not None:
        _lib.need(workspace.dtype == torch.uint8 and workspace.is_contiguous(),
                  f"{what}: workspace must be contiguous uint8")


def select_workspace_bytes(m, n_q_heads, n_kv_heads, window_blocks, block_size):
    """Bytes of the workspace nkv_compress_select needs."""
    return _lib.lib().nkv_compress_select_workspace_bytes(m, n_q_heads, n_kv_heads,
                                                          window_blocks, block_size)


def compress_select(q, k_cache, block_tables, base_context_lens, seq_idx, window_blocks,
                    num_keep, scale, agg="all", importance=None, keep_idx=None, workspace=None):
    """Score the window of each selected sequence and pick the kept positions.

    A caller-provided ``workspace`` is uint8 of >= select_workspace_bytes(...).
    Returns (keep_idx int32 [m, n_sets, 1+num_keep+1], importance fp32
    [m, n_sets, W*B-1]). keep_idx rows are [0, ascending top-num_keep, W*B-1].
    """
    m = seq_idx.numel()
    NB, B, Hk, D = k_cache.shape
    Hq = q.size(1)
    n_sets = 1 if agg == "all" else Hk
    n_cand = window_blocks * B - 1
    _check_window_args("compress_select", q, k_cache, None, block_tables, base_context_lens, None,
                       seq_idx, importance, keep_idx, workspace, n_sets, n_cand, num_keep + 2)
    L = _lib.lib()
    if importance is None:
        importance = torch.empty(m, n_sets, n_cand, dtype=torch.float32, device=q.device)
    if keep_idx is None:
        keep_idx = torch.empty(m, n_sets, num_keep + 2, dtype=torch.int32, device=q.device)
    ws_bytes = select_workspace_bytes(m, Hq, Hk, window_blocks, B)
    if workspace is None:
        workspace = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=q.device)
    fn = L.nkv_compress_select_f16 if q.dtype == torch.float16 else L.nkv_compress_select
    rc = fn(
        q.data_ptr(), q.stride(0), k_cache.data_ptr(), block_tables.data_ptr(),
        block_tables.stride(0), block_tables.size(1), base_context_lens.data_ptr(),
        seq_idx.data_ptr(), m, Hq, Hk, D, B, window_blocks, NB, float(scale), AGG_MODES[agg],
        num_keep, importance.data_ptr(), keep_idx.data_ptr(), workspace.data_ptr(),
        workspace.numel(), _lib.stream_of(q))
    _lib.check(rc, "compress_select")
    return keep_idx, importance


def compress_compact(k_cache, v_cache, block_tables, base_context_lens, context_lens, seq_idx,
                     keep_idx, window_blocks):
    """Move the kept window rows (and the tail block) into place, K and V."""
    NB, B, Hk, D = k_cache.shape
    m, n_sets, keep_tokens = keep_idx.shape
    _check_window_args("compress_compact", None, k_cache, v_cache, block_tables,
                       base_context_lens, context_lens, seq_idx, None, keep_idx, None, n_sets,
                       None, keep_tokens)
    _lib.need(m == seq_idx.numel(), "compress_compact: keep_idx needs one row per seq_idx entry")
    rc = _lib.lib().nkv_compress_compact(
        k_cache.data_ptr(), v_cache.data_ptr(), block_tables.data_ptr(), block_tables.stride(0),
        block_tables.size(1), base_context_lens.data_ptr(), context_lens.data_ptr(),
        seq_idx.data_ptr(), m, keep_idx.data_ptr(), n_sets, keep_tokens, Hk, D, B,
        window_blocks, NB, _lib.stream_of(k_cache))
    _lib.check(rc, "compress_compact")


def compress_step(q, k_cache, v_cache, block_tables, base_context_lens, context_lens, seq_idx,
                  window_blocks, keep_tokens, scale, agg="all", importance=None, keep_idx=None,
                  workspace=None, k_scale=1.0, events=None, rewrite_tables=True,
                  slot_mapping=None):
    """compress_select + compress_compact in one call (fused on the GPU).

    Returns (keep_idx, importance) like compress_select; the caches and
    context_lens are updated like compress_compact. With ``events`` (the last
    layer) the call also does compress_finalize's bookkeeping (events, table
    and slot rewrite), inside the fused launch.
    """
    m = seq_idx.numel()
    NB, B, Hk, D = k_cache.shape
    Hq = q.size(1)
    n_sets = 1 if agg == "all" else Hk
    n_cand = window_blocks * B - 1
    _check_window_args("compress_step", q, k_cache, v_cache, block_tables, base_context_lens,
                       context_lens, seq_idx, importance, keep_idx, workspace, n_sets, n_cand,
                       keep_tokens)
    if importance is None:
        importance = torch.empty(m, n_sets, n_cand, dtype=torch.float32, device=q.device)
    if keep_idx is None:
        keep_idx = torch.empty(m, n_sets, keep_tokens, dtype=torch.int32, device=q.device)
    ws_bytes = select_workspace_bytes(m, Hq, Hk, window_blocks, B)
    if workspace is None:
        workspace = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=q.device)
    fin = []  # the bookkeeping's arguments, appended to the step's
    if events is not None:
        _check_finalize_args(block_tables, base_context_lens, seq_idx, events, slot_mapping)
        fin = [int(bool(rewrite_tables)), _lib.ptr(slot_mapping), events.data_ptr()]
    name = "nkv_compress_step" + ("_finalize" if fin else "")
    if k_cache.dtype == torch.float8_e4m3fn:  # fp8 pool (K read as code * k_scale)
        name += "_fp8"
        rc = getattr(_lib.lib(), name)(
            q.data_ptr(), q.stride(0), k_cache.data_ptr(), v_cache.data_ptr(),
            block_tables.data_ptr(), block_tables.stride(0), block_tables.size(1),
            base_context_lens.data_ptr(), context_lens.data_ptr(), seq_idx.data_ptr(), m, Hq, Hk,
            D, B, window_blocks, NB, float(scale), float(k_scale), AGG_MODES[agg], keep_tokens,
            importance.data_ptr(), keep_idx.data_ptr(), workspace.data_ptr(), workspace.numel(),
            *fin, _lib.stream_of(q))
        _lib.check(rc, name[4:])
        return keep_idx, importance
    if q.dtype == torch.float16:
        name += "_f16"
    rc = getattr(_lib.lib(), name)(
        q.data_ptr(), q.stride(0), k_cache.data_ptr(), v_cache.data_ptr(), block_tables.data_ptr(),
        block_tables.stride(0), block_tables.size(1), base_context_lens.data_ptr(),
        context_lens.data_ptr(), seq_idx.data_ptr(), m, Hq, Hk, D, B, window_blocks, NB,
        float(scale), AGG_MODES[agg], keep_tokens, importance.data_ptr(), keep_idx.data_ptr(),
        workspace.data_ptr(), workspace.numel(), *fin, _lib.stream_of(q))
    _lib.check(rc, name[4:])
    return keep_idx, importance


def _check_finalize_args(block_tables, base_context_lens, seq_idx, events, slot_mapping):
    _lib.require_device(block_tables.device, base_context_lens=base_context_lens,
                        seq_idx=seq_idx, events=events, slot_mapping=slot_mapping)
    _lib.need(all(t.dtype == torch.int32 for t in (block_tables, base_context_lens, seq_idx,
                                                   events)),
              "compress_finalize: tables, lengths, seq_idx and events must be int32")
    _lib.need(slot_mapping is None or slot_mapping.dtype == torch.int32,
              "compress_finalize: slot_mapping must be int32")
    _lib.need(events.is_contiguous() and events.numel() >= seq_idx.numel() *
              (4 + block_tables.size(1)),
              "compress_finalize: events needs [m, 4 + max_blocks] int32 entries")


def compress_finalize(block_tables, base_context_lens, seq_idx, keep_tokens, block_size,
                      window_blocks, events, rewrite_tables=True, slot_mapping=None):
    _check_finalize_args(block_tables, base_context_lens, seq_idx, events, slot_mapping)
    rc = _lib.lib().nkv_compress_finalize(
        block_tables.data_ptr(), block_tables.stride(0), block_tables.size(1),
        base_context_lens.data_ptr(), seq_idx.data_ptr(), seq_idx.numel(), keep_tokens,
        block_size, window_blocks, int(bool(rewrite_tables)), _lib.ptr(slot_mapping),
        events.data_ptr(), _lib.stream_of(block_tables))
    _lib.check(rc, "compress_finalize")


def events_to_dicts(events: torch.Tensor, layer_id: int) -> list[dict]:
    """Decode the int32 event rows into the reference's event dicts (:280-287).

    Padding rows (batch index -1) give no dict. A row with n_freed = -1 is a selected
    sequence that was not compressible (fewer than W full blocks, or a table too short):
    the reference asserts there (:39-41); here it is left unchanged and its dict carries
    ``skipped: True``, which apply_compression_events ignores."""
    out = []
    for row in events.cpu().tolist():
        if row[0] < 0:
            continue
        n = row[3]
        ev = {
            "batch_index": int(row[0]),
            "layer": int(layer_id),
            "new_context_len": int(row[1]),
            "keep_blocks": int(row[2]),
            "freed_block_ids": [int(x) for x in row[4:4 + max(n, 0)]],
            "tail_uncompressed_len_after": 0,
        }
        if n < 0:
            ev["skipped"] = True
        out.append(ev)
    return out


def MyCompressCompact(q_current: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                      layer_id: int, block_size: int, window_blocks: int, keep_blocks: int,
                      keep_extra_tokens: int, num_layers: int, context=None, agg: str = "all",
                      rewrite_tables: bool = True, k_scale: float = 1.0) -> bool:
    """Compress the last ``window_blocks`` full blocks of each selected sequence.

    agg="all" sums key importance over every query head (the reference,
    CompressMethod.py:41-42); agg="group" keeps a separate set per KV head.
    A selected sequence whose base length has fewer than ``window_blocks``
    full blocks is left unchanged (the reference asserts instead, :39-41).
    """
    if context is None:
        from ..utils.context import get_context
        context = get_context()
    if (not context.use_decode_kernel) or context.context_lens is None \
            or context.block_tables is None:
        return False
    device_sel = getattr(context, "compress_seq_idx", None)
    if device_sel is not None:  # selected on the device (nkv_compress_schedule), -1 padded
        selected = device_sel
        m = selected.numel()
    else:
        selected = context.compress_selected_batch_indices
        if not selected:
            return False
        m = len(selected)
        bs = context.context_lens.numel()
        assert all(0 <= i < bs for i in selected) and len(set(selected)) == m, \
            f"selected batch indices must be distinct and < {bs}: {selected}"
    B = block_size
    window_tokens = window_blocks * B
    keep_tokens = keep_blocks * B + keep_extra_tokens
    num_keep = keep_tokens - 2  # bos + selected + latest token
    # SnapKV's own skip rule with window = 1 (CompressMethod.py:17-18)
    if window_tokens - 1 <= 0 or window_tokens <= num_keep + 1:
        return False
    base = context.compress_base_context_lens
    assert base is not None, "compress_base_context_lens is None during compress step"
    device = k_cache.device
    Hq, D = q_current.size(1), q_current.size(2)
    Hk = k_cache.size(2)
    n_sets = 1 if agg == "all" else Hk
    ws_bytes = select_workspace_bytes(m, Hq, Hk, window_blocks, B)
    buf = _buffers(context, selected, device, m, n_sets, window_tokens - 1, keep_tokens,
                   ws_bytes, 4 + context.block_tables.size(1))
    last = layer_id + 1 >= num_layers  # the last layer also does the bookkeeping (:266-288)
    compress_step(q_current, k_cache, v_cache, context.block_tables, base, context.context_lens,
                  buf.seq_idx, window_blocks, keep_tokens, D ** -0.5, agg,
                  importance=buf.importance, keep_idx=buf.keep_idx, workspace=buf.workspace,
                  k_scale=k_scale, events=buf.events if last else None,
                  rewrite_tables=rewrite_tables,
                  slot_mapping=context.slot_mapping if rewrite_tables else None)
    if last:
        if device_sel is not None:  # read by the host after the step, no sync here
            context.compression_events_device = buf.events
        else:
            if context.compression_events is None:
                context.compression_events = []
            context.compression_events.extend(events_to_dicts(buf.events, layer_id))
    return True


def compress_schedule(context_lens, tail_uncompressed, block_size, window_blocks, topk, period,
                      step_counter, seq_idx, n_selected, base_context_lens=None,
                      policy="first"):
    """The compression selection of prepare_decode (model_runner.py:300-332) on the device:
    advances ``step_counter`` and fills ``seq_idx`` (int32 [topk], -1 padded),
    ``n_selected`` and ``base_context_lens`` without reading anything on the host."""
    bs = context_lens.numel()
    assert tail_uncompressed.numel() >= bs and seq_idx.numel() == topk
    _lib.require_device(context_lens.device, tail_uncompressed=tail_uncompressed,
                        step_counter=step_counter, seq_idx=seq_idx, n_selected=n_selected,
                        base_context_lens=base_context_lens)
    rc = _lib.lib().nkv_compress_schedule(
        context_lens.data_ptr(), tail_uncompressed.data_ptr(), bs, block_size, window_blocks,
        topk, period, {"first": 0, "longest": 1}[policy], step_counter.data_ptr(),
        seq_idx.data_ptr(), n_selected.data_ptr(), _lib.ptr(base_context_lens),
        _lib.stream_of(context_lens))
    _lib.check(rc, "compress_schedule")
