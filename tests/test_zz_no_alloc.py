"""nkv_paged_decode_noalloc (the decode entry point that allocates nothing) through the C ABI:
bitwise equal to nkv_paged_decode with a caller workspace, on two calls in a row (the
second smaller, so it runs over the first call's leftovers in the fixed array), within
2e-2 of the fp32 oracle, and a request beyond the array's size rejected before launching.
"""
import importlib

import pytest
import torch

from oracle.attention_ref import paged_decode_ref

pytestmark = pytest.mark.gpu
wl_mod = importlib.import_module("nanokv-llm_amd.workloads")
L = importlib.import_module("nanokv-llm_amd._lib")
EUNSUPPORTED = -4


def _both(dev, wl):
    """(out of nkv_paged_decode with a workspace, out of nkv_paged_decode_noalloc)."""
    lib = L.lib()
    q, kc, vc = wl["q"].to(dev), wl["k_cache"].to(dev), wl["v_cache"].to(dev)
    bt, ctx = wl["block_tables"][0].to(dev), wl["context_lens"].to(dev)
    bs, Hq, D = q.shape
    NB, B, Hk, _ = kc.shape
    width = bt.size(1)
    sh = L.stream_of(q)
    ws = torch.empty(lib.nkv_paged_decode_workspace_bytes(bs, Hq, D, width, B),
                     dtype=torch.uint8, device=dev)
    ref_out = torch.empty(bs, Hq, D, dtype=torch.bfloat16, device=dev)
    L.check(lib.nkv_paged_decode(q.data_ptr(), q.stride(0), kc.data_ptr(), vc.data_ptr(),
                                 bt.data_ptr(), bt.stride(0), ctx.data_ptr(), bs, Hq, Hk, D, B,
                                 width, NB, wl["scale"], ref_out.data_ptr(), ref_out.stride(0),
                                 ws.data_ptr(), ws.numel(), sh), "paged_decode")
    out = torch.full((bs, Hq, D), 7.0, dtype=torch.bfloat16, device=dev)
    L.check(lib.nkv_paged_decode_noalloc(q.data_ptr(), q.stride(0), kc.data_ptr(),
                                         vc.data_ptr(), bt.data_ptr(), bt.stride(0),
                                         ctx.data_ptr(), bs, Hq, Hk, D, B, width, NB,
                                         wl["scale"], out.data_ptr(), out.stride(0), sh),
            "paged_decode_noalloc")
    torch.cuda.synchronize()
    return ref_out, out


def test_noalloc_equals_workspace_entry_point_twice(dev):
    # first call: Qwen3-8B geometry, 48 sequences of up to 6000 tokens (two heads per wave)
    big = wl_mod.decode_workload(48, 32, 8, 1000, 6000, 48 * 24 + 8, seed=71)
    # second call, smaller: 5 sequences, Qwen3-14B grouping (g = 5), one head per wave
    small = wl_mod.decode_workload(5, 40, 8, 1, 900, 5 * 4 + 4, seed=72)
    for name, wl in (("first (48 x 32 heads)", big), ("second (5 x 40 heads)", small)):
        print(f"no-alloc decode, {name}", flush=True)
        ref_out, out = _both(dev, wl)
        assert torch.equal(out, ref_out), name
        ref = paged_decode_ref(wl["q"].float(), wl["k_cache"], wl["v_cache"],
                               wl["context_lens"], wl["block_tables"][0], wl["scale"])
        assert (out.float().cpu() - ref).abs().max().item() <= 2e-2, name


def test_noalloc_rejects_beyond_the_array(dev):
    """4000 sequences x 64 query heads need more partial rows than the 64 MiB array holds:
    refused on the host with NKV_EUNSUPPORTED, the output left as it was."""
    lib = L.lib()
    bs, Hq, Hk, D, B = 4000, 64, 8, 128, 256
    q = torch.zeros(bs, Hq, D, dtype=torch.bfloat16, device=dev)
    kc = torch.zeros(2, B, Hk, D, dtype=torch.bfloat16, device=dev)
    bt = torch.zeros(bs, 1, dtype=torch.int32, device=dev)
    ctx = torch.ones(bs, dtype=torch.int32, device=dev)
    out = torch.full((bs, Hq, D), 3.0, dtype=torch.bfloat16, device=dev)
    rc = lib.nkv_paged_decode_noalloc(q.data_ptr(), q.stride(0), kc.data_ptr(), kc.data_ptr(),
                                      bt.data_ptr(), 1, ctx.data_ptr(), bs, Hq, Hk, D, B, 1, 2,
                                      D ** -0.5, out.data_ptr(), out.stride(0), L.stream_of(q))
    assert rc == EUNSUPPORTED and b"array" in lib.nkv_last_error()
    torch.cuda.synchronize()
    assert bool((out == 3.0).all())
