"""The fp8 (OCP E4M3FN) oracle pinned on the CPU: torch's float8_e4m3fn decode against the
format's definition for all 256 codes, and its rounding against a brute-force nearest-even
search over every finite bf16 input; clamping, NaN and the store's slot rules."""
import torch

from oracle import fp8_ref


def test_decode_table_matches_definition():
    table = fp8_ref.e4m3fn_table()
    tv = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).double()
    assert torch.equal(torch.isnan(table), torch.isnan(tv))
    ok = ~torch.isnan(table)
    assert torch.equal(table[ok], tv[ok])
    assert table[0x7E].item() == 448.0 and table[0x01].item() == 2.0 ** -9


def test_encode_matches_brute_force_on_every_bf16():
    x = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    f = x.float()
    fin = torch.isfinite(f) & (f.abs() <= 448)
    assert torch.equal(fp8_ref.fp8_quantize_ref(x[fin]), fp8_ref.nearest_e4m3fn(f[fin]))
    big = torch.isfinite(f) & (f.abs() > 448)
    codes = fp8_ref.fp8_quantize_ref(x[big])
    assert set(codes.tolist()) == {0x7E, 0xFE}  # clamped to +-448
    assert set(fp8_ref.fp8_quantize_ref(x[torch.isnan(f)]).tolist()) <= {0x7F, 0xFF}


def test_round_trip_and_planted_error():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(4096, generator=g).to(torch.bfloat16)
    y = fp8_ref.fp8_dequantize_ref(fp8_ref.fp8_quantize_ref(x, 0.5), 0.5)
    normal = x.float().abs() * 2 >= 2 ** -6  # scaled value in E4M3FN's normal range
    rel = ((y.float() - x.float()).abs() / x.float().abs())[normal].max().item()
    assert rel <= 2 ** -4  # 3 mantissa bits: half an ulp is at most 2^-4 relative
    tiny = ~normal  # subnormal spacing 2^-9 of the scaled value: absolute error <= 2^-11
    assert (y.float() - x.float()).abs()[tiny].max().item() <= 2 ** -11
    # truncation instead of rounding (a plausible mistake) fails the brute-force check
    trunc = (x.float().abs() * 8).floor() / 8
    assert not torch.equal(fp8_ref.nearest_e4m3fn(trunc * torch.sign(x.float())),
                           fp8_ref.nearest_e4m3fn(x.float()))


def test_store_fp8_ref_slots():
    g = torch.Generator().manual_seed(2)
    key = torch.randn(5, 2, 16, generator=g).to(torch.bfloat16)
    value = torch.randn(5, 2, 16, generator=g).to(torch.bfloat16)
    kc = torch.zeros(2, 4, 2, 16, dtype=torch.uint8)
    vc = torch.zeros_like(kc)
    slots = torch.tensor([3, -1, 0, 7, 5], dtype=torch.int32)
    fp8_ref.store_kvcache_fp8_ref(key, value, kc, vc, slots, 2.0, 0.5)
    kf = kc.view(-1, 32)
    assert torch.equal(kf[3], fp8_ref.fp8_quantize_ref(key[0].reshape(-1), 2.0))
    assert torch.equal(kf[1], torch.zeros(32, dtype=torch.uint8))  # untouched
    assert torch.equal(vc.view(-1, 32)[7], fp8_ref.fp8_quantize_ref(value[3].reshape(-1), 0.5))
