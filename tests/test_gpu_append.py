"""HIP RoPE / cache-write entry points vs the oracle, bit for bit, and the
engine-API mirror (RopeCache, KVCache, apply_rope, apply_flash_decoding) run
as the reference's per-token decode loop."""
import numpy as np
import pytest
import torch

from lucciola_rs_amd import workloads as wl
from lucciola_rs_amd.engine import KVCache, apply_flash_decoding, apply_rope, sm_scale
from gpu_util import TOL, from_dev, rope_cache, say, to_dev
import pins

pytestmark = pytest.mark.gpu


def make_rows(rng, n, hq, hkv, d, dtype):
    row = (hq + 2 * hkv) * d
    qkv = pins.bits(rng.standard_normal((n, row)) * 0.6, dtype)
    qb = pins.bits(rng.standard_normal(hq * d) * 0.2, dtype)
    kb = pins.bits(rng.standard_normal(hkv * d) * 0.2, dtype)
    vb = pins.bits(rng.standard_normal(hkv * d) * 0.2, dtype)
    return qkv, qb, kb, vb


@pytest.mark.parametrize("pad", [0, 2], ids=["vec", "padded"])
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("hq,hkv,d", [(14, 2, 64), (28, 4, 128), (12, 2, 128)])
def test_rope_append_bit_exact(orc, luc, dtype, hq, hkv, d, pad):
    """pad=0: 16-byte aligned rows (the 16-byte chunk kernel); pad=2: a row
    stride of row + 2 elements (the element-wise kernel).  Both bit-exact."""
    rng = np.random.default_rng(hq + d)
    positions = np.array([0, 1, 15, 16, 17, 31, 32, 255, 256, 511, 4095, 639], np.int32)
    n = len(positions)
    # every row (sequence) owns its pages, so no two rows share a cache slot
    L, layer, pages = 3, 1, n * 40 + 1
    qkv, qb, kb, vb = make_rows(rng, n, hq, hkv, d, dtype)
    if pad:  # padding columns the kernels must leave alone
        qkv = np.concatenate([qkv, pins.bits(rng.standard_normal((n, pad)), dtype)], axis=1)
    perm = rng.permutation(pages - 1).astype(np.int32)
    tables = np.full((n, 256), pages - 1, np.int32)
    tables[:, :40] = perm.reshape(n, 40)
    tables[10, 255] = tables[10, 39]  # position 4095 -> logical page 255
    kp = pins.bits(rng.standard_normal((pages, L, hkv, 16, d)), dtype)
    vp = pins.bits(rng.standard_normal((pages, L, hkv, 16, d)), dtype)
    rope = rope_cache(luc, d)
    cos, sin = rope.cos.cpu().numpy(), rope.sin.cpu().numpy()

    # oracle: rope then cache write, row by row (models.rs:505-534)
    oq, ok_, ov = qkv.copy(), kp.copy(), vp.copy()
    qd, kd = hq * d, hkv * d
    for r in range(n):
        row = oq[r]
        qv, kv, vv = row[:qd], row[qd:qd + kd], row[qd + kd:qd + 2 * kd]
        q2, k2 = qv.copy(), kv.copy()
        orc.rope(q2, qb, k2, kb, cos, sin, int(positions[r]), d, hq, hkv, dtype)
        row[:qd], row[qd:qd + kd] = q2, k2
        orc.kv_update(ok_, ov, k2, np.ascontiguousarray(vv), vb, np.ascontiguousarray(tables[r]),
                      layer, int(positions[r]), L, hkv, d, 16, dtype)

    t_qkv, t_kp, t_vp = to_dev(qkv, dtype), to_dev(kp, dtype), to_dev(vp, dtype)
    t_tab = torch.from_numpy(tables).cuda()
    t_pos = torch.from_numpy(positions).cuda()
    bq, bk, bv = to_dev(qb, dtype), to_dev(kb, dtype), to_dev(vb, dtype)
    say(f"  [gpu] rope_append {dtype} hq={hq} hkv={hkv} d={d} rows={n}")
    luc.rope_append(t_qkv, bq, t_qkv[:, qd:], bk, t_qkv[:, qd + kd:], bv, qkv.shape[1], rope.cos,
                    rope.sin, t_pos, t_tab, t_kp, t_vp, n, layer, L, hq, hkv, d)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(t_qkv), oq)
    assert np.array_equal(from_dev(t_kp), ok_)
    assert np.array_equal(from_dev(t_vp), ov)

    # the two separate entry points give the same bits
    t_qkv, t_kp, t_vp = to_dev(qkv, dtype), to_dev(kp, dtype), to_dev(vp, dtype)
    say("  [gpu] rope + kv_cache_update")
    luc.rope(t_qkv, bq, t_qkv[:, qd:], bk, qkv.shape[1], rope.cos, rope.sin, t_pos, n, hq, hkv, d)
    luc.kv_cache_update(t_kp, t_vp, t_qkv[:, qd:], t_qkv[:, qd + kd:], bv, qkv.shape[1], t_tab,
                        t_pos, n, layer, L, hkv, d)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(t_qkv), oq)
    assert np.array_equal(from_dev(t_kp), ok_)
    assert np.array_equal(from_dev(t_vp), ov)


def special_values(rng, shape, dtype):
    """A mix that exercises every rounding path of the rotation: ordinary
    values, values whose rotated results are subnormal, values near the top of
    the range (sums overflow to inf), infinities, NaNs, signed zeros."""
    big = 3.0e38 if dtype == "bf16" else 6.0e4
    tiny = 1.0e-39 if dtype == "bf16" else 3.0e-6
    n = int(np.prod(shape))
    kind = rng.integers(0, 8, n)
    x = rng.standard_normal(n)
    x = np.where(kind == 1, x * tiny, x)
    x = np.where(kind == 2, np.sign(x) * big * rng.uniform(0.5, 1.0, n), x)
    x = np.where(kind == 3, np.inf * np.sign(x), x)
    x = np.where(kind == 4, np.nan, x)
    x = np.where(kind == 5, np.copysign(0.0, x), x)
    b = pins.bits(x.reshape(shape), dtype)
    # NaNs with other payloads and signs, set bit by bit
    nan = rng.random(b.shape) < 0.02
    payload = (0x7fc1 if dtype == "bf16" else 0x7e01) | (rng.integers(0, 2, b.shape) << 15)
    return np.where(nan, payload, b).astype(np.uint16)


@pytest.mark.parametrize("pad", [0, 2], ids=["vec", "padded"])
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_rope_append_special_values_bit_exact(orc, luc, dtype, pad):
    """Subnormal results, overflow to inf, inf/NaN inputs and signed zeros:
    the GPU rotation and rounding match the oracle bit for bit (NaN results:
    NaN on both sides), through the 16-byte chunk kernel (pad=0) and the
    element-wise one (pad=2)."""
    rng = np.random.default_rng(77)
    hq, hkv, d = 14, 2, 64
    n = 24
    positions = rng.integers(0, 4096, n).astype(np.int32)
    row = (hq + 2 * hkv) * d
    qkv = special_values(rng, (n, row + pad), dtype)
    qb = special_values(rng, (hq * d,), dtype)
    kb = pins.bits(rng.standard_normal(hkv * d) * 0.2, dtype)
    vb = special_values(rng, (hkv * d,), dtype)
    L, layer, pages = 1, 0, n * 256 + 1
    tables = (np.arange(n * 256, dtype=np.int32).reshape(n, 256))
    kp = np.zeros((pages, L, hkv, 16, d), np.uint16)
    vp = np.zeros((pages, L, hkv, 16, d), np.uint16)
    rope = rope_cache(luc, d)
    cos, sin = rope.cos.cpu().numpy(), rope.sin.cpu().numpy()
    oq, ok_, ov = qkv.copy(), kp.copy(), vp.copy()
    qd, kd = hq * d, hkv * d
    for r in range(n):
        rw = oq[r]
        q2, k2 = rw[:qd].copy(), rw[qd:qd + kd].copy()
        orc.rope(q2, qb, k2, kb, cos, sin, int(positions[r]), d, hq, hkv, dtype)
        rw[:qd], rw[qd:qd + kd] = q2, k2
        orc.kv_update(ok_, ov, k2, np.ascontiguousarray(rw[qd + kd:qd + 2 * kd]), vb,
                      np.ascontiguousarray(tables[r]), layer, int(positions[r]), L, hkv, d, 16, dtype)
    t_qkv, t_kp, t_vp = to_dev(qkv, dtype), to_dev(kp, dtype), to_dev(vp, dtype)
    say(f"  [gpu] rope_append special values {dtype} pad={pad}")
    luc.rope_append(t_qkv, to_dev(qb, dtype), t_qkv[:, qd:], to_dev(kb, dtype), t_qkv[:, qd + kd:],
                    to_dev(vb, dtype), qkv.shape[1], rope.cos, rope.sin,
                    torch.from_numpy(positions).cuda(), torch.from_numpy(tables).cuda(), t_kp, t_vp,
                    n, layer, L, hq, hkv, d)
    torch.cuda.synchronize()
    # IEEE 754 leaves the sign and payload of a NaN that arithmetic produces
    # unspecified (x86 and the GPU propagate them differently): NaN must meet
    # NaN, every other value its exact bits
    top = 0x7c00 if dtype == "f16" else 0x7f80
    for name, got, want in (("qkv", from_dev(t_qkv), oq), ("k_pool", from_dev(t_kp), ok_),
                            ("v_pool", from_dev(t_vp), ov)):
        gnan, wnan = (got & 0x7fff) > top, (want & 0x7fff) > top
        bad = np.argwhere((got != want) & ~(gnan & wnan))
        assert bad.size == 0, (f"{name}: {len(bad)} differ, first at {bad[:4].tolist()}: "
                               f"got {[hex(v) for v in got[tuple(bad[:4].T)]]} "
                               f"want {[hex(v) for v in want[tuple(bad[:4].T)]]}")


def test_engine_api_decode_loop(orc, luc):
    """The reference's single-sequence loop through the engine mirror: for
    pos in 0..S-1, apply_rope -> KVCache.update -> apply_flash_decoding
    (src/models.rs:485-550), against the oracle doing the same."""
    hq, hkv, d, L, S, dtype = 14, 2, 64, 2, 300, "bf16"
    rng = np.random.default_rng(77)
    qkv, qb, kb, vb = make_rows(rng, S, hq, hkv, d, dtype)
    rope = rope_cache(luc, d)
    cos, sin = rope.cos.cpu().numpy(), rope.sin.cpu().numpy()
    cache = KVCache(L, hkv, d, num_physical_blocks=40, max_position_embeddings=1024,
                    dtype=torch.bfloat16, lib=luc)
    layer = 1
    t_qkv = to_dev(qkv, dtype).reshape(-1)
    out = torch.zeros(S * hq * d, dtype=torch.bfloat16, device="cuda")
    bq, bk, bv = to_dev(qb, dtype), to_dev(kb, dtype), to_dev(vb, dtype)
    pos_dev = torch.zeros(1, dtype=torch.int32, device="cuda")
    row = (hq + 2 * hkv) * d
    say(f"  [gpu] engine loop S={S}")
    for t in range(S):
        pos_dev.fill_(t)
        off = t * row
        apply_rope(rope, t_qkv, off, off + hq * d, bq, bk, pos_dev, d, hq, hkv, lib=luc)
        cache.update(layer, t, pos_dev, t_qkv[off + hq * d:], t_qkv[off + (hq + hkv) * d:], bv)
        apply_flash_decoding(out, t * hq * d, t_qkv, off, cache, layer, t, pos_dev, d, hq, hkv,
                             lib=luc)
    torch.cuda.synchronize()
    # the table was handed out LIFO: 0, 1, 2, ... (kv_cache.rs:73-76)
    assert cache.block_table_cpu == list(range((S + 15) // 16))

    table = np.asarray(cache.block_table_cpu + [0] * 4, np.int32)
    kp = np.zeros((40, L, hkv, 16, d), np.uint16)
    vp = np.zeros_like(kp)
    oq = qkv.copy()
    want = orc.prefill(oq, qb, kb, vb, cos, sin, kp, vp, table[None].copy(),
                       np.array([0, S], np.int32), np.array([0], np.int32), layer, hq, hkv, d,
                       sm_scale(d), 16, L, dtype)
    assert np.array_equal(from_dev(t_qkv).reshape(S, row), oq)
    assert np.array_equal(from_dev(cache.k_pool), kp)
    assert np.array_equal(from_dev(cache.v_pool), vp)
    got = pins.f32(from_dev(out), dtype).reshape(S, hq, d)
    err = float(np.max(np.abs(got - pins.f32(want, dtype))))
    say(f"  max|hip - oracle| = {err:.3e}")
    assert err <= TOL[dtype]


def test_kv_cache_out_of_blocks(luc):
    cache = KVCache(1, 2, 64, num_physical_blocks=2, max_position_embeddings=64, lib=luc)
    cache.prepare_for_step(0)
    cache.prepare_for_step(16)
    with pytest.raises(RuntimeError, match="Out of memory blocks"):
        cache.prepare_for_step(32)


def test_append_skips_positions_outside_table(orc, luc):
    """A position past the table row is not written anywhere."""
    dtype, hq, hkv, d = "f16", 2, 1, 64
    rng = np.random.default_rng(1)
    qkv, _, _, _ = make_rows(rng, 2, hq, hkv, d, dtype)
    kp = pins.bits(rng.standard_normal((4, 1, hkv, 16, d)), dtype)
    t_kp, t_vp = to_dev(kp, dtype), to_dev(kp, dtype)
    t_qkv = to_dev(qkv, dtype)
    tables = torch.tensor([[1, 2], [3, 0]], dtype=torch.int32, device="cuda")
    pos = torch.tensor([32, -1], dtype=torch.int32, device="cuda")  # table holds 32 slots
    rope = rope_cache(luc, d)
    say("  [gpu] rope_append out-of-table positions")
    luc.rope_append(t_qkv, None, t_qkv[:, hq * d:], None, t_qkv[:, (hq + hkv) * d:], None,
                    qkv.shape[1], rope.cos, rope.sin, pos, tables, t_kp, t_vp, 2, 0, 1, hq, hkv, d)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(t_kp), kp) and np.array_equal(from_dev(t_vp), kp)
    assert np.array_equal(from_dev(t_qkv), qkv)
