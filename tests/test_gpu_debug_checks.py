"""The input checks of the debug build (libnkv_amd_debug.so, NKV_DEBUG) on the GPU.

The kernels skip or clamp inputs the reference would stop on or access out of bounds
with: a slot past the pool (store), a needed block-table entry outside the pool (decode,
prefill, compression scoring), a context longer than its table row (decode), a rotary
position past the cos/sin table. The debug build does exactly what the release build does
with them and also records one NKV_DEBUG_* bit per kind, read back with nkv_debug_flags.
Checks: clean inputs record nothing; each bad input records exactly the bits it should;
every output equals the release library's bit for bit. Every input here is one the
kernels' own bounds checks turn into a skip, a zero read or a clamp.
"""
import ctypes as C
import importlib

import pytest
import torch

pytestmark = pytest.mark.gpu
L = importlib.import_module("nanokv-llm_amd._lib")
W = importlib.import_module("nanokv-llm_amd.workloads")
cu = importlib.import_module("nanokv-llm_amd.layers.compress_utils")
SLOT, BLOCK, LENGTH, POSITION = (L.NKV_DEBUG_SLOT, L.NKV_DEBUG_BLOCK, L.NKV_DEBUG_LENGTH,
                                 L.NKV_DEBUG_POSITION)


@pytest.fixture(scope="module")
def dbg(nkv):
    h = C.CDLL(L.DEBUG_LIB_PATH)
    for name, (res, args) in L.SIGNATURES.items():
        fn = getattr(h, name)
        fn.restype, fn.argtypes = res, args
    return h


def _flags(h):
    v = C.c_uint32(0)
    assert h.nkv_debug_flags(C.addressof(v), 1) == 0, h.nkv_last_error()
    return v.value


def _both(monkeypatch, dbg, fn):
    """fn() through the release library, then through the debug one; returns both results
    and the bits the debug run recorded."""
    rel = fn()
    torch.cuda.synchronize()
    _flags(dbg)  # start clean
    with monkeypatch.context() as m:
        m.setattr(L, "_LIB", dbg)
        deb = fn()
    return rel, deb, _flags(dbg)


def _equal(a, b):
    if isinstance(a, (tuple, list)):
        return all(_equal(x, y) for x, y in zip(a, b))
    return torch.equal(a, b)


def test_store_slots(nkv, dev, dbg, monkeypatch):
    g = torch.Generator().manual_seed(11)
    N, Hk, D, NB, B = 8, 8, 128, 2, 256
    key = torch.randn(N, Hk, D, generator=g).to(torch.bfloat16).to(dev)
    value = torch.randn(N, Hk, D, generator=g).to(torch.bfloat16).to(dev)
    base = torch.randn(NB, B, Hk, D, generator=g).to(torch.bfloat16).to(dev)
    for slots, bits in (([0, 5, -1, 511, 200, 7, 9, 3], 0),
                        ([0, 5, -1, 511, 512, -7, 1000, 3], SLOT)):
        sl = torch.tensor(slots, dtype=torch.int32, device=dev)

        def run():
            kc, vc = base.clone(), base.clone()
            nkv.store_kvcache(key, value, kc, vc, sl)
            return kc, vc

        rel, deb, got = _both(monkeypatch, dbg, run)
        assert got == bits
        assert _equal(rel, deb)


def test_decode_blocks_and_lengths(nkv, dev, dbg, monkeypatch):
    wl = W.decode_workload(4, 16, 8, 300, 1000, 16, seed=12)
    q, kc, vc = wl["q"].to(dev), wl["k_cache"].to(dev), wl["v_cache"].to(dev)
    bt0 = wl["block_tables"][0]
    ctx0 = wl["context_lens"]
    n_blocks, B = kc.size(0), kc.size(1)
    bad_bt = bt0.clone()
    bad_bt[1, 0] = -1            # a needed block missing
    bad_bt[2, 1] = n_blocks + 3  # and one past the pool
    long_ctx = ctx0.clone()
    # longer than the table row covers: clamped to the row, whose padding entries past the
    # sequence's own blocks are then needed as well
    long_ctx[0] = bt0.size(1) * B + 10
    assert int((bt0[0] < 0).sum()) > 0
    for bt, ctx, bits in ((bt0, ctx0, 0), (bad_bt, ctx0, BLOCK),
                          (bt0, long_ctx, LENGTH | BLOCK)):
        def run():
            return nkv.paged_decode(q, kc, vc, ctx.to(dev), bt.to(dev), wl["scale"])

        rel, deb, got = _both(monkeypatch, dbg, run)
        assert got == bits
        assert _equal(rel, deb)


def test_prefill_blocks(nkv, dev, dbg, monkeypatch):
    wl = W.prefill_workload(3, 16, 8, 100, 700, seed=13, device=dev)
    bt0 = wl["block_tables"]
    bad = bt0.clone()
    bad[1, 0] = -1
    for bt, bits in ((bt0, 0), (bad, BLOCK)):
        def run():
            return nkv.varlen_prefill(wl["q"], wl["k_cache"], wl["v_cache"],
                                      wl["cu_seqlens_q"].to(dev), wl["cu_seqlens_k"].to(dev),
                                      wl["max_seqlen_q"], wl["scale"], block_tables=bt.to(dev),
                                      max_seqlen_k=wl["max_seqlen_k"])

        rel, deb, got = _both(monkeypatch, dbg, run)
        assert got == bits
        assert _equal(rel, deb)


def test_rope_positions_and_slots(nkv, dev, dbg, monkeypatch):
    g = torch.Generator().manual_seed(14)
    N, Hq, Hk, D, max_pos = 6, 16, 8, 128, 64
    q = torch.randn(N, Hq, D, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(N, Hk, D, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(N, Hk, D, generator=g).to(torch.bfloat16).to(dev)
    cs = torch.randn(max_pos, D, generator=g).to(dev)
    base = torch.randn(1, 16, Hk, D, generator=g).to(torch.bfloat16).to(dev)
    good_pos = [0, 5, 63, 7, 8, 9]
    for pos, slots, bits in ((good_pos, [0, 1, 2, -1, 4, 5], 0),
                             ([0, 5, 64, -2, 8, 9], [0, 1, 2, -1, 4, 5], POSITION),
                             (good_pos, [0, 1, 16, -1, -3, 5], SLOT)):
        p = torch.tensor(pos, dtype=torch.int64, device=dev)
        sl = torch.tensor(slots, dtype=torch.int32, device=dev)

        def run():
            kc, vc = base.clone(), base.clone()
            qo, ko, _ = nkv.qk_norm_rope_store(p, q, k, v, cs, k_cache=kc, v_cache=vc,
                                               slot_mapping=sl)
            return qo, ko, kc, vc

        rel, deb, got = _both(monkeypatch, dbg, run)
        assert got == bits
        assert _equal(rel, deb)


def test_compression_scoring_blocks(nkv, dev, dbg, monkeypatch):
    wl = W.compress_workload(6, 16, 8, 1100, 1600, 2, seed=15, device=dev, selected_only=True)
    sel = torch.tensor(wl["seq_idx"], dtype=torch.int32, device=dev)
    ctx = wl["context_lens"].to(dev)
    bt0 = wl["block_tables"]
    bad = bt0.clone()
    s = wl["seq_idx"][0]
    full = int(wl["context_lens"][s]) // 256
    bad[s, full - 1] = -1  # a window block of the first selected sequence
    for bt, bits in ((bt0, 0), (bad, BLOCK)):
        def run():
            keep, imp = cu.compress_select(wl["q"].to(dev), wl["k_cache"], bt.to(dev), ctx, sel,
                                           4, 511, 128 ** -0.5, agg="group")
            return keep, imp

        rel, deb, got = _both(monkeypatch, dbg, run)
        assert got == bits
        assert _equal(rel, deb)
