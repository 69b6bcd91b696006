"""The last layer's compression step with its bookkeeping in the same launch
(nkv_compress_step_finalize and its f16 / fp8 forms) against the two launches it
replaces (nkv_compress_step, then nkv_compress_finalize, whose events, tables and slots
the oracle pins in test_gpu_compress.py): importance, kept sets, caches, context_lens,
events, block tables and slot maps bit for bit.

Covered: both aggregations; bf16, fp16 and fp8 pools; -1 padding entries and a selected
sequence that cannot be compressed; rewrite_tables off and no slot map; table rows with
more than 128 entries past the kept blocks (the bookkeeping's own loads); shapes the
fused kernels do not take (GQA group 32, 2048-token windows), where the bookkeeping
follows as its own launch; consecutive calls with other sizes (the arrival counters
return to zero), one of them with more workgroups than the GPU has CUs.
"""
import importlib

import pytest
import torch

pytestmark = pytest.mark.gpu
wl_mod = importlib.import_module("nanokv-llm_amd.workloads")
cu = importlib.import_module("nanokv-llm_amd.layers.compress_utils")

W = 4


def _pool(kc, vc, dtype):
    if dtype == "fp16":
        return kc.to(torch.float16), vc.to(torch.float16)
    if dtype == "fp8":  # N(0, 1) values: every one inside the E4M3 range
        return kc.float().to(torch.float8_e4m3fn), vc.float().to(torch.float8_e4m3fn)
    return kc, vc


def _run(dev, q, kc, vc, bt, lens, sel, agg, keep, B, fused, rewrite=True, slots=True,
         k_scale=1.0):
    kg, vg = kc.to(dev), vc.to(dev)
    btg = bt.to(dev)
    base = lens.to(dev)
    ctx = base.clone()
    seq_idx = torch.tensor(sel, dtype=torch.int32, device=dev)
    events = torch.full((len(sel), 4 + bt.size(1)), 77, dtype=torch.int32, device=dev)
    slot = (torch.arange(bt.size(0), dtype=torch.int32, device=dev) * 3 + 1) if slots else None
    D = q.size(-1)
    kw = dict(events=events, rewrite_tables=rewrite, slot_mapping=slot) if fused else {}
    keep_idx, imp = cu.compress_step(q.to(dev), kg, vg, btg, base, ctx, seq_idx, W, keep,
                                     D ** -0.5, agg, k_scale=k_scale, **kw)
    if not fused:
        cu.compress_finalize(btg, base, seq_idx, keep, B, W, events, rewrite_tables=rewrite,
                             slot_mapping=slot)
    torch.cuda.synchronize()
    out = dict(keep=keep_idx, imp=imp, k=kg, v=vg, ctx=ctx, events=events, bt=btg)
    if slot is not None:
        out["slot"] = slot
    return {n: t.cpu() for n, t in out.items()}


def _check_equal(a, b):
    assert a.keys() == b.keys()
    for name in a:
        if name in ("keep", "imp"):  # padding rows are left unwritten
            continue
        x, y = a[name], b[name]
        if x.dtype == torch.float8_e4m3fn:
            x, y = x.view(torch.uint8), y.view(torch.uint8)
        assert torch.equal(x, y), f"{name} differs"


def _compare(dev, q, kc, vc, bt, lens, sel, agg, keep, B, **kw):
    print(f"fused finalize: m={len(sel)} Hq={q.size(1)} Hk={kc.size(2)} B={B} agg={agg} "
          f"dtype={kc.dtype} {kw}", flush=True)
    two = _run(dev, q, kc, vc, bt, lens, sel, agg, keep, B, False, **kw)
    one = _run(dev, q, kc, vc, bt, lens, sel, agg, keep, B, True, **kw)
    _check_equal(two, one)
    rows = [r for r, s in enumerate(sel) if s >= 0]
    for name in ("keep", "imp"):
        assert torch.equal(two[name][rows], one[name][rows]), f"{name} differs"
    return one


def _state(seed, bs=48, Hq=32, Hk=8, topk=10):
    wl = wl_mod.compress_workload(bs, Hq, Hk, 1500, 4096, topk, seed, selected_only=True)
    return wl["q"], wl["k_cache"], wl["v_cache"], wl["block_tables"], wl["context_lens"], \
        list(wl["seq_idx"])


@pytest.mark.parametrize("dtype", ["bf16", "fp16", "fp8"])
@pytest.mark.parametrize("agg", ["all", "group"])
def test_fused_finalize_equals_two_launches(nkv, dev, agg, dtype):
    q, kc, vc, bt, lens, sel = _state(21)
    lens = lens.clone()
    short = sel[3]
    lens[short] = 3 * 256 + 40  # fewer than W full blocks: left unchanged, n_freed -1
    sel = sel[:5] + [-1] + sel[5:] + [-1, -1]  # padding rows read [-1, 0, 0, 0, -1...]
    if dtype == "fp16":
        q = q.to(torch.float16)
    kc, vc = _pool(kc, vc, dtype)
    one = _compare(dev, q, kc, vc, bt, lens, sel, agg, 2 * 256 + 1, 256,
                   k_scale=0.5 if dtype == "fp8" else 1.0)
    ev = one["events"]
    assert ev[5, :4].tolist() == [-1, 0, 0, 0] and torch.all(ev[5, 4:] == -1)
    assert ev[3, 0] == short and ev[3, 3] == -1  # skipped
    assert all(int(ev[r, 3]) >= 1 for r, s in enumerate(sel) if s >= 0 and s != short)


def test_fused_finalize_rewrite_off_and_no_slots(nkv, dev):
    q, kc, vc, bt, lens, sel = _state(22, topk=6)
    one = _compare(dev, q, kc, vc, bt, lens, sel, "group", 2 * 256 + 1, 256, rewrite=False,
                   slots=False)
    assert torch.equal(one["bt"], bt)


@pytest.mark.parametrize("agg", ["all", "group"])
def test_fused_finalize_long_table_rows(nkv, dev, agg):
    """Rows of 151 and 200 blocks, and a row whose entries past its 5 blocks hold 190 more
    ids (every id >= 0 past the kept blocks is freed): 192 freed ids run over the two
    entries per lane read ahead into the bookkeeping's own loop."""
    B, Hk, G, D = 256, 2, 2, 128
    lens = [150 * B + 30, W * B + 7, 200 * B, 5 * B + 255]
    g = torch.Generator().manual_seed(23)
    width = 205
    n_blocks = sum((n + B - 1) // B for n in lens) + 4
    perm = torch.randperm(n_blocks, generator=g).tolist()
    rows = []
    for n in lens:
        nb = (n + B - 1) // B
        rows.append([perm.pop() for _ in range(nb)] + [-1] * (width - nb))
    rows[1][5:195] = [10000 + i for i in range(190)]
    bt = torch.tensor(rows, dtype=torch.int32)
    kc = torch.randn(n_blocks, B, Hk, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(n_blocks, B, Hk, D, generator=g).to(torch.bfloat16)
    q = torch.randn(len(lens), Hk * G, D, generator=g).to(torch.bfloat16)
    lt = torch.tensor(lens, dtype=torch.int32)
    one = _compare(dev, q, kc, vc, bt, lt, [0, 1, 2, 3], agg, 2 * B + 1, B)
    ev = one["events"]
    assert ev[0, 2:4].tolist() == [149, 2]  # 151 blocks, 149 kept
    assert ev[1, 2:4].tolist() == [3, 192]
    assert ev[1, 4:196].tolist() == [int(x) for x in rows[1][3:195]]
    assert ev[2, 2:4].tolist() == [199, 1]


def test_fused_finalize_general_path(nkv, dev):
    """Group 32 (above the fused kernels' 16 MFMA rows) and a 2048-token window: the
    step takes the multi-kernel path and the bookkeeping runs as its own launch."""
    q, kc, vc, bt, lens, sel = _state(24, bs=24, Hq=64, Hk=2, topk=5)
    _compare(dev, q, kc, vc, bt, lens, sel, "group", 2 * 256 + 1, 256)
    B = 512
    wl = wl_mod.compress_workload(16, 8, 2, 2100, 4096, 4, 25, selected_only=True)
    # a pool of 512-token blocks for the same lengths
    g = torch.Generator().manual_seed(25)
    lens = wl["context_lens"]
    n_blocks = sum((int(n) + B - 1) // B for n in lens) + 2
    perm = torch.randperm(n_blocks, generator=g).tolist()
    width = max((int(n) + B - 1) // B for n in lens) + 1
    rows = []
    for n in lens.tolist():
        nb = (n + B - 1) // B
        rows.append([perm.pop() for _ in range(nb)] + [-1] * (width - nb))
    bt = torch.tensor(rows, dtype=torch.int32)
    kc = torch.randn(n_blocks, B, 2, 128, generator=g).to(torch.bfloat16)
    vc = torch.randn(n_blocks, B, 2, 128, generator=g).to(torch.bfloat16)
    sel = [i for i in range(16) if int(lens[i]) >= W * B][:4]
    assert sel
    _compare(dev, wl["q"], kc, vc, bt, lens, sel, "all", 2 * B + 1, B)


def test_fused_finalize_consecutive_calls(nkv, dev):
    """Calls in a row with other sizes: 40 sequences x 8 KV heads (320 workgroups, more
    than the CUs), then 7 x 4, 3 x 1 (one unit per sequence: every arrival is the last),
    then 12 x 8; each equals the two launches."""
    for seed, bs, Hk, topk in ((26, 80, 8, 40), (27, 20, 4, 7), (29, 8, 1, 3), (28, 30, 8, 12)):
        q, kc, vc, bt, lens, sel = _state(seed, bs=bs, Hq=4 * Hk, Hk=Hk, topk=topk)
        _compare(dev, q, kc, vc, bt, lens, sel, "group" if Hk in (8, 1) else "all", 2 * 256 + 1,
                 256)
