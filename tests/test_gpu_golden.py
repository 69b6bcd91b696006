"""The HIP path against the golden fixtures of tests/golden/ (through the C ABI).

Floating point: max abs err <= 2e-2 (bf16 outputs vs fp32 expected); importance
within rtol 1e-4. Integer and byte results bit-exact.
"""
import importlib

import numpy as np
import pytest
import torch

from golden_util import digest, events_array, from_bits, load
from oracle.compress_ref import select_topk_ref

pytestmark = pytest.mark.gpu
TOL = 2e-2
W, KEEP = 4, 2 * 256 + 1
wl_mod = importlib.import_module("nanokv-llm_amd.workloads")
cu = importlib.import_module("nanokv-llm_amd.layers.compress_utils")


def test_decode_golden(nkv, dev):
    fx = load("decode_qwen3_0_6b.npz")
    wl = wl_mod.decode_qwen3_0_6b(seed=1)
    kg, vg = wl["k_cache"].to(dev), wl["v_cache"].to(dev)
    slots = torch.from_numpy(fx["slot_mapping"]).to(dev)
    nkv.store_kvcache(wl["key"].to(dev), wl["value"].to(dev), kg, vg, slots)
    out = nkv.paged_decode(wl["q"].to(dev), kg, vg, torch.from_numpy(fx["context_lens"]).to(dev),
                           torch.from_numpy(fx["block_tables"]).to(dev), float(fx["scale"]))
    torch.cuda.synchronize()
    assert np.abs(out.float().cpu().numpy() - fx["out"]).max() <= TOL


def test_prefill_golden(nkv, dev):
    fx = load("prefill_small.npz")
    q, kc, vc = from_bits(fx["q"]), from_bits(fx["k_cache"]), from_bits(fx["v_cache"])
    out = nkv.varlen_prefill(q.to(dev), kc.to(dev), vc.to(dev),
                             torch.from_numpy(fx["cu_seqlens_q"]).to(dev),
                             torch.from_numpy(fx["cu_seqlens_k"]).to(dev), int(fx["max_seqlen_q"]),
                             float(fx["scale"]),
                             block_tables=torch.from_numpy(fx["block_tables"]).to(dev))
    torch.cuda.synchronize()
    assert np.abs(out.float().cpu().numpy() - fx["out"]).max() <= TOL


@pytest.mark.parametrize("agg", ["all", "group"])
def test_compress_select_golden(nkv, dev, agg):
    fx = load("compress_small.npz")
    wl = wl_mod.compress_workload(6, 8, 2, 1100, 2000, 2, 11, selected_only=True)
    sel = torch.from_numpy(fx["seq_idx"]).to(dev)
    keep, imp = cu.compress_select(wl["q"].to(dev), wl["k_cache"].to(dev),
                                   torch.from_numpy(fx["block_tables"]).to(dev),
                                   torch.from_numpy(fx["context_lens"]).to(dev), sel, W,
                                   KEEP - 2, 128 ** -0.5, agg)
    torch.cuda.synchronize()
    imp = imp.cpu()
    assert np.allclose(imp.numpy(), fx[f"importance_{agg}"], rtol=1e-4, atol=1e-7)
    got = keep.cpu()
    # bit-exact given identical scores, and (near-ties aside) the fixture's sets
    assert torch.equal(got[..., 1:-1].long(), select_topk_ref(imp, KEEP - 2))
    exp = fx[f"keep_{agg}"]
    for r in range(exp.shape[0]):
        for s in range(exp.shape[1]):
            a, b = set(got[r, s].tolist()), set(exp[r, s].tolist())
            assert len(a & b) / len(b) >= 0.99


def test_compress_compact_golden(nkv, dev):
    fx = load("compress_small.npz")
    wl = wl_mod.compress_workload(6, 8, 2, 1100, 2000, 2, 11, selected_only=True)
    kg, vg = wl["k_cache"].to(dev), wl["v_cache"].to(dev)
    btg = torch.from_numpy(fx["block_tables"]).to(dev)
    base = torch.from_numpy(fx["context_lens"]).to(dev)
    ctx = base.clone()
    sel = torch.from_numpy(fx["seq_idx"]).to(dev)
    keep = torch.from_numpy(fx["keep_all"]).to(dev)
    cu.compress_compact(kg, vg, btg, base, ctx, sel, keep, W)
    width = btg.size(1)
    events = torch.empty(sel.numel(), 4 + width, dtype=torch.int32, device=dev)
    slots = torch.full((btg.size(0),), -1, dtype=torch.int32, device=dev)
    cu.compress_finalize(btg, base, sel, KEEP, 256, W, events, rewrite_tables=True,
                         slot_mapping=slots)
    torch.cuda.synchronize()
    assert digest(kg.cpu()) == str(fx["digest_k_after"])
    assert digest(vg.cpu()) == str(fx["digest_v_after"])
    assert np.array_equal(ctx.cpu().numpy(), fx["context_lens_after"])
    assert np.array_equal(events_array(cu.events_to_dicts(events, 0), width), fx["events"])
    assert np.array_equal(btg.cpu().numpy(), fx["block_tables_after"])
    got_slots = slots.cpu().numpy()
    s_idx = fx["seq_idx"]
    assert np.array_equal(got_slots[s_idx], fx["next_slot"][s_idx])


def test_compress_step_golden(nkv, dev):
    """The fused step (agg "all") reproduces the fixture's compaction when its kept sets
    equal the fixture's (they do unless fp32 near-ties reorder the threshold)."""
    fx = load("compress_small.npz")
    wl = wl_mod.compress_workload(6, 8, 2, 1100, 2000, 2, 11, selected_only=True)
    kg, vg = wl["k_cache"].to(dev), wl["v_cache"].to(dev)
    btg = torch.from_numpy(fx["block_tables"]).to(dev)
    base = torch.from_numpy(fx["context_lens"]).to(dev)
    ctx = base.clone()
    sel = torch.from_numpy(fx["seq_idx"]).to(dev)
    keep, imp = cu.compress_step(wl["q"].to(dev), kg, vg, btg, base, ctx, sel, W, KEEP,
                                 128 ** -0.5, "all")
    torch.cuda.synchronize()
    assert np.allclose(imp.cpu().numpy(), fx["importance_all"], rtol=1e-4, atol=1e-7)
    assert np.array_equal(ctx.cpu().numpy(), fx["context_lens_after"])
    if np.array_equal(keep.cpu().numpy(), fx["keep_all"]):
        assert digest(kg.cpu()) == str(fx["digest_k_after"])
        assert digest(vg.cpu()) == str(fx["digest_v_after"])
