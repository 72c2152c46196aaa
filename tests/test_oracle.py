"""The oracle against independent checks (CPU only)."""
import numpy as np
import pytest
import torch

import pins


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_conversion_roundtrip_all_bit_patterns(orc, dtype):
    # every 16-bit pattern -> f32 -> 16-bit is the identity (NaNs stay NaN)
    allb = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = orc.to_f32(allb, dtype)
    want = pins.f32(allb, dtype)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(f), nan)
    assert np.array_equal(f[~nan].view(np.uint32), want[~nan].view(np.uint32))
    back = orc.to_storage(f, dtype)
    assert np.array_equal(back[~nan], allb[~nan])


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_conversion_rne_matches_torch(orc, dtype):
    # random f32 bit patterns across the whole range, plus exact halfway cases
    rng = np.random.default_rng(0)
    u = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    if dtype == "bf16":
        half = (rng.integers(0, 2**16, 100_000).astype(np.uint32) << 16) | 0x8000
    else:
        # f16 halfway points: f16 value + half an f16 ulp, normal and subnormal ranges
        h = rng.integers(1, 0x7bff, 100_000).astype(np.uint16)
        lo = pins.f32(h, "f16").astype(np.float64)
        hi = pins.f32(h + 1, "f16").astype(np.float64)
        half = ((lo + hi) / 2).astype(np.float32).view(np.uint32)
    x = np.concatenate([u, half]).view(np.float32)
    x = x[~np.isnan(x)]
    got = orc.to_storage(x, dtype)
    want = pins.bits(x, dtype)
    assert np.array_equal(got, want)


def test_rope_table_closed_form(orc):
    assert pins.check_rope_table(orc) <= 1.0
    assert pins.check_rope_table(orc, head_dim=128, max_pos=1024) <= 1.0
    assert pins.check_rope_table(orc, scale=4.0, max_pos=512) <= 1.0


def test_rope_table_position_zero_and_head_dim(orc):
    cos, sin = orc.rope_table(4, 64, 1e6)
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)
    # i = 0 has inverse frequency 1: theta = pos exactly
    assert cos[3, 0] == np.float32(np.cos(np.float32(3.0)))


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_rope_rotation(orc, dtype, head_dim):
    assert pins.check_rope(orc, dtype, head_dim) <= 1.0
    assert pins.check_rope(orc, dtype, head_dim, with_bias=False, seed=4) <= 1.0


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_rope_position_zero_is_identity(orc, dtype):
    rng = np.random.default_rng(2)
    cos, sin = orc.rope_table(8, 64, 1e6)
    q = pins.bits(rng.standard_normal((14, 64)), dtype)
    k = pins.bits(rng.standard_normal((2, 64)), dtype)
    q2, k2 = q.copy(), k.copy()
    orc.rope(q2, None, k2, None, cos, sin, 0, 64, 14, 2, dtype)
    assert np.array_equal(q2, q) and np.array_equal(k2, k)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_kv_update_slots(orc, dtype):
    assert pins.check_kv_update(orc, dtype) == 0
    assert pins.check_kv_update(orc, dtype, num_layers=1, hkv=4, head_dim=128, seed=3) == 0


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("ctx", [1, 2, 16, 17, 31, 32, 33, 100, 512, 1500])
def test_attention_vs_f64(orc, dtype, ctx):
    assert pins.check_attention(orc, dtype, ctx, seed=ctx) <= 1.0


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_attention_head128_gqa_layers(orc, dtype):
    assert pins.check_attention(orc, dtype, 700, hq=28, hkv=4, head_dim=128, layer=2,
                                num_layers=3) <= 1.0
    assert pins.check_attention(orc, dtype, 300, hq=12, hkv=2, head_dim=128) <= 1.0


def test_attention_outliers(orc):
    assert pins.check_attention(orc, "bf16", 2000, hq=12, hkv=2, head_dim=128,
                                outliers=0.01) <= 1.0


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_attention_vs_torch_sdpa(orc, dtype):
    assert pins.check_attention_sdpa(orc, dtype, 333) <= 1.0
    assert pins.check_attention_sdpa(orc, dtype, 64, hq=28, hkv=4, head_dim=128) <= 1.0


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_attention_invariants(orc, dtype):
    assert pins.check_attention_invariants(orc, dtype) == 0
    assert pins.check_attention_invariants(orc, dtype, head_dim=128) == 0


def test_attention_empty_context_is_nan(orc):
    # pos = -1: no token; the reference's merge divides 0 by 0
    q, kp, vp, table = pins.attention_inputs("bf16", 1, 2, 1, 64, 3, 0)
    out = orc.flash_decoding(q, kp, vp, table, 0, 2, 1, 64, -1, 0.125, 16, 1, "bf16")
    assert np.all(np.isnan(pins.f32(out, "bf16")))


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_prefill_causal(orc, dtype):
    assert pins.check_prefill(orc, dtype) <= 1.0


def test_decode_batch_equals_single(orc):
    # batched application == the single-sequence function per sequence
    rng = np.random.default_rng(9)
    B, hq, hkv, d, pool = 3, 14, 2, 64, 40
    kp = pins.bits(rng.standard_normal((pool, 2, hkv, 16, d)), "f16")
    vp = pins.bits(rng.standard_normal((pool, 2, hkv, 16, d)), "f16")
    tables = rng.permutation(pool).astype(np.int32)[:36].reshape(B, 12).copy()
    pos = np.array([5, 191, 77], np.int32)
    q = pins.bits(rng.standard_normal((B, hq, d)), "f16")
    out = orc.decode_batch(q, kp, vp, tables, pos, 1, hq, hkv, d, 0.125, 16, 2, "f16")
    for b in range(B):
        one = orc.flash_decoding(np.ascontiguousarray(q[b]), kp, vp, np.ascontiguousarray(tables[b]),
                                 1, hq, hkv, d, int(pos[b]), 0.125, 16, 2, "f16")
        assert np.array_equal(out[b], one)


def test_rmsnorm_vs_f64(orc):
    assert pins.check_rmsnorm(orc) <= 1


def test_silu_mul_vs_f64(orc):
    assert pins.check_silu_mul(orc) <= 1


def test_argmax_first_of_equals_nan_and_floor(orc):
    assert pins.check_argmax(orc) == 0


def test_oracle_qwen2_loop_vs_f64_decoder(orc):
    assert pins.check_oracle_model(orc) <= 1


def test_topk_filter_matches_closed_form(orc):
    """Candidates of the 32-partition filter: keys and value bits equal the
    closed-form order (value, then the reference's tree tie order), with NaN,
    -inf, values <= -1e30, signed zeros and a short partition."""
    assert pins.check_topk_filter(orc) == 0


def test_bitonic_network_matches_recursive_form(orc):
    assert pins.check_bitonic(orc) == 0


def test_top_p_pick_matches_f64_closed_form(orc):
    assert pins.check_top_p(orc) == 0
