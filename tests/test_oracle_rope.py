"""The norm + rope oracle pinned on the CPU.

Checks: Hugging Face transformers' Qwen3 implementation (Qwen3RMSNorm,
Qwen3RotaryEmbedding, apply_rotary_pos_emb) as an independent library
routine for the same maths, bit-for-bit; the rotation's invariants (pair norms
kept, identity at position 0, scores depend only on the position offset); and
a planted sign error that those checks catch.
"""
import pytest
import torch

from oracle import rope_ref
from oracle.attention_ref import store_kvcache_ref

hf = pytest.importorskip("transformers.models.qwen3.modeling_qwen3")
from transformers import Qwen3Config  # noqa: E402

D = 128


def _hf_rotary(max_pos, base):
    cfg = Qwen3Config(head_dim=D, hidden_size=4096, num_attention_heads=32,
                      num_key_value_heads=8, rope_theta=base, max_position_embeddings=max_pos)
    return hf.Qwen3RotaryEmbedding(cfg)


@pytest.mark.parametrize("base", [10000.0, 1000000.0])
def test_cos_sin_cache_matches_hf(base):
    cache = rope_ref.rotary_cos_sin_cache_ref(D, 4096, base)
    pos = torch.arange(4096)[None]
    cos, sin = _hf_rotary(4096, base)(torch.zeros(1, 1, D), pos)
    assert torch.equal(cache[:, :64], cos[0, :, :64]) and torch.equal(cache[:, 64:], sin[0, :, :64])
    # HF's table repeats the half: the rotation pairs element j with j + 64
    assert torch.equal(cos[0, :, :64], cos[0, :, 64:])


def test_rms_norm_matches_hf():
    g = torch.Generator().manual_seed(1)
    x = (torch.randn(64, 8, D, generator=g) * 3).to(torch.bfloat16)
    w = (1 + 0.3 * torch.randn(D, generator=g)).to(torch.bfloat16)
    norm = hf.Qwen3RMSNorm(D, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(w.float())
    norm = norm.to(torch.bfloat16)
    with torch.no_grad():
        assert torch.equal(rope_ref.rms_norm_ref(x, w, 1e-6), norm(x))


def test_rotary_matches_hf():
    g = torch.Generator().manual_seed(2)
    N, Hq, Hk = 50, 32, 8
    q = torch.randn(N, Hq, D, generator=g)
    k = torch.randn(N, Hk, D, generator=g)
    pos = torch.randint(0, 40000, (N,), generator=g)
    cache = rope_ref.rotary_cos_sin_cache_ref(D, 40960, 1e6)
    qr, kr = rope_ref.rotary_ref(pos, q, k, cache)
    cos, sin = _hf_rotary(40960, 1e6)(torch.zeros(1, 1, D), pos[None])
    qh, kh = hf.apply_rotary_pos_emb(q, k, cos[0], sin[0], unsqueeze_dim=1)
    assert torch.equal(qr, qh) and torch.equal(kr, kh)


def test_rotary_invariants():
    g = torch.Generator().manual_seed(3)
    cache = rope_ref.rotary_cos_sin_cache_ref(D, 8192, 1e6)
    x = torch.randn(16, 4, D, generator=g, dtype=torch.float32)
    pos = torch.randint(0, 8192, (16,), generator=g)
    y, _ = rope_ref.rotary_ref(pos, x, x[:, :1], cache)
    pair = lambda t: t[..., :64].double() ** 2 + t[..., 64:].double() ** 2  # noqa: E731
    assert torch.allclose(pair(y), pair(x), rtol=1e-5, atol=1e-6)
    y0, _ = rope_ref.rotary_ref(torch.zeros(16, dtype=torch.long), x, x[:, :1], cache)
    assert torch.equal(y0, x)
    # <R_m q, R_n k> depends on m - n only
    q, k = x[:1], x[1:2]
    s = []
    for m, n in [(100, 40), (1100, 1040), (5060, 5000)]:
        qm, _ = rope_ref.rotary_ref(torch.tensor([m]), q, q[:, :1], cache)
        kn, _ = rope_ref.rotary_ref(torch.tensor([n]), k, k[:, :1], cache)
        s.append((qm.double() * kn.double()).sum().item())
    assert max(s) - min(s) < 1e-3 * (1 + abs(s[0]))


def test_planted_sign_error_is_caught():
    """The same rotation with the second half's sign flipped fails the HF check."""
    g = torch.Generator().manual_seed(4)
    x = torch.randn(8, 2, D, generator=g)
    cache = rope_ref.rotary_cos_sin_cache_ref(D, 512, 1e6)
    pos = torch.randint(1, 512, (8,), generator=g)
    cs = cache[pos].unsqueeze(1)
    cos, sin = cs.chunk(2, dim=-1)
    x1, x2 = x.chunk(2, dim=-1)
    wrong = torch.cat((x1 * cos - x2 * sin, x2 * cos - x1 * sin), dim=-1)
    c2, s2 = _hf_rotary(512, 1e6)(torch.zeros(1, 1, D), pos[None])
    good, _ = hf.apply_rotary_pos_emb(x, x, c2[0], s2[0], unsqueeze_dim=1)
    assert not torch.allclose(wrong, good, atol=1e-3)
    assert torch.equal(rope_ref.apply_rotary_ref(x, cos, sin), good)


def test_fused_ref_composes_the_steps():
    """qkv split + norm + rope + store equals the steps run one by one."""
    g = torch.Generator().manual_seed(5)
    N, Hq, Hk = 12, 4, 2
    qkv = torch.randn(N, (Hq + 2 * Hk) * D, generator=g).to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    cache = rope_ref.rotary_cos_sin_cache_ref(D, 1024, 1e6)
    pos = torch.randint(0, 1024, (N,), generator=g)
    kc = torch.zeros(4, 16, Hk, D, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    slots = torch.randperm(64, generator=g)[:N].to(torch.int32)
    slots[3] = -1
    q, k, v = rope_ref.qk_norm_rope_store_ref(qkv, pos, qw, kw, 1e-6, cache, Hq, Hk,
                                              k_cache=kc, v_cache=vc, slot_mapping=slots)
    qs = qkv[:, :Hq * D].reshape(N, Hq, D)
    ks = qkv[:, Hq * D:(Hq + Hk) * D].reshape(N, Hk, D)
    vs = qkv[:, (Hq + Hk) * D:].reshape(N, Hk, D)
    q2, k2 = rope_ref.rotary_ref(pos, rope_ref.rms_norm_ref(qs, qw, 1e-6),
                                 rope_ref.rms_norm_ref(ks, kw, 1e-6), cache)
    assert torch.equal(q, q2) and torch.equal(k, k2) and torch.equal(v, vs)
    kc2, vc2 = torch.zeros_like(kc), torch.zeros_like(vc)
    store_kvcache_ref(k2, vs, kc2, vc2, slots)
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)
    assert kc.view(-1, Hk * D).abs().sum(-1).gt(0).sum().item() == N - 1
