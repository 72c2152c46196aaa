"""Independent checks that pin the oracle (oracle/luc_oracle.c).

Each check computes the same quantity a different way -- f64 closed forms,
a textbook attention in numpy float64, torch's scaled_dot_product_attention,
or an index computed from a numpy reshape of the pool -- and returns the worst
error relative to its tolerance (<= 1 passes).  The checks are written so a
plausible mistake in the oracle (a dropped term, a wrong sign or index, a
swapped operand) exceeds the tolerance; tests/test_oracle_mutants.py builds
such mistakes into the oracle and confirms each check catches them.
"""
from __future__ import annotations

import numpy as np
import torch

PAGE = 16


def ulp(x: np.ndarray, dtype: str) -> np.ndarray:
    """Spacing of the 16-bit storage format at |x| (subnormal floor included)."""
    mant = 10 if dtype == "f16" else 7
    emin = -14 if dtype == "f16" else -126
    a = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** emin)))
    return 2.0 ** (e - mant)


def store(x, dtype):
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    return t.to(torch.float16 if dtype == "f16" else torch.bfloat16).float().numpy()


def bits(x, dtype):
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    return t.to(torch.float16 if dtype == "f16" else torch.bfloat16).view(
        torch.int16).numpy().view(np.uint16)


def f32(b, dtype):
    t = torch.from_numpy(np.ascontiguousarray(b).view(np.int16))
    return t.view(torch.float16 if dtype == "f16" else torch.bfloat16).float().numpy()


# ---------------------------------------------------------------- RoPE table
def check_rope_table(orc, max_pos=4096, head_dim=64, base=1e6, scale=None):
    """Table vs the f64 closed form theta = (pos/scale) / base^(2i/d).
    f32 evaluation of theta (a pow, two divides) is within a few f32 ulp of
    the exact theta; cos/sin are then within |theta| * 2^-21 + 2^-23."""
    cos, sin = orc.rope_table(max_pos, head_dim, base, scale)
    pos = np.arange(max_pos, dtype=np.float64)[:, None]
    i = np.arange(head_dim // 2, dtype=np.float64)[None, :]
    s = scale or 1.0
    theta = (pos / s) / np.power(float(np.float32(base)), 2 * i / head_dim)
    tol = np.abs(theta) * 2.0 ** -21 + 2.0 ** -23
    err = np.maximum(np.abs(cos - np.cos(theta)), np.abs(sin - np.sin(theta)))
    return float(np.max(err / tol))


# ---------------------------------------------------------------- RoPE apply
def check_rope(orc, dtype, head_dim=64, hq=14, hkv=2, seed=0, with_bias=True):
    """Apply the oracle's rope at random positions; compare with the f64
    rotation of (x + bias) by the table's own cos/sin, rounded once."""
    rng = np.random.default_rng(seed)
    cos, sin = orc.rope_table(2048, head_dim, 1e6)
    worst = 0.0
    for pos in [0, 1, 15, 16, 17, 511, 2047] + list(rng.integers(0, 2048, 5)):
        q = bits(rng.standard_normal((hq, head_dim)) * 0.7, dtype)
        k = bits(rng.standard_normal((hkv, head_dim)) * 0.7, dtype)
        qb = bits(rng.standard_normal((hq, head_dim)) * 0.3, dtype) if with_bias else None
        kb = bits(rng.standard_normal((hkv, head_dim)) * 0.3, dtype) if with_bias else None
        q2, k2 = q.copy(), k.copy()
        orc.rope(q2, qb, k2, kb, cos, sin, int(pos), head_dim, hq, hkv, dtype)
        for x, b, got in ((q, qb, q2), (k, kb, k2)):
            xv = f32(x, dtype).astype(np.float64)
            if b is not None:
                xv = xv + f32(b, dtype)
            h = head_dim // 2
            c = cos[pos].astype(np.float64)
            s = sin[pos].astype(np.float64)
            want = np.concatenate([xv[:, :h] * c - xv[:, h:] * s, xv[:, :h] * s + xv[:, h:] * c],
                                  axis=1)
            g = f32(got, dtype).astype(np.float64)
            # f32 products/sums then one rounding: <= 1 storage ulp (+ f32 slack)
            tol = ulp(want, dtype) * 1.01 + np.abs(want) * 2.0 ** -22 + 1e-30
            worst = max(worst, float(np.max(np.abs(g - want) / tol)))
    return worst


# ------------------------------------------------------------ cache slots
def check_kv_update(orc, dtype, num_layers=3, hkv=2, head_dim=64, pool=20, seed=0):
    """Write tagged tokens through orc_kv_update and read the pool back with
    a numpy view [page][layer][head][slot][dim]: every written slot holds its
    token (K bit-exact, V = round(v + bias)); every other slot is untouched.
    Returns the number of wrong entries."""
    rng = np.random.default_rng(seed)
    table = rng.permutation(pool).astype(np.int32)[:8]  # 8 pages -> 128 positions
    shape = (pool, num_layers, hkv, PAGE, head_dim)
    sentinel = bits(np.full(shape, 3.0), dtype)
    kp, vp = sentinel.copy(), sentinel.copy()
    written = {}
    positions = [0, 1, 14, 15, 16, 17, 31, 32, 33, 47, 48, 100, 127]
    vb = bits(rng.standard_normal((hkv, head_dim)), dtype)
    for layer in range(num_layers):
        for pos in positions:
            k = bits(rng.standard_normal((hkv, head_dim)), dtype)
            v = bits(rng.standard_normal((hkv, head_dim)), dtype)
            orc.kv_update(kp, vp, k, v, vb, table, layer, pos, num_layers, hkv, head_dim, PAGE,
                          dtype)
            written[(layer, pos)] = (k, v)
    bad = 0
    expect_k, expect_v = sentinel.copy(), sentinel.copy()
    for (layer, pos), (k, v) in written.items():
        page, slot = table[pos // PAGE], pos % PAGE
        expect_k[page, layer, :, slot, :] = k
        expect_v[page, layer, :, slot, :] = bits(
            f32(v, dtype).astype(np.float64) + f32(vb, dtype), dtype)
    bad += int(np.count_nonzero(kp != expect_k))
    bad += int(np.count_nonzero(vp != expect_v))
    # the closed-form slot offset agrees with the numpy view
    for pos in positions:
        for layer in range(num_layers):
            for h in range(hkv):
                off = orc.slot_offset(table, pos, layer, h, num_layers, hkv, head_dim, PAGE)
                idx = np.ravel_multi_index((table[pos // PAGE], layer, h, pos % PAGE, 0), shape)
                bad += int(off != idx)
    return bad


# ------------------------------------------------------------- attention
def gather_kv(k_pool, v_pool, table, layer, kv_head, ctx, dtype):
    pages = table[: (ctx + PAGE - 1) // PAGE]
    k = f32(k_pool[pages, layer, kv_head].reshape(-1, k_pool.shape[-1])[:ctx], dtype)
    v = f32(v_pool[pages, layer, kv_head].reshape(-1, v_pool.shape[-1])[:ctx], dtype)
    return k.astype(np.float64), v.astype(np.float64)


def textbook_attention(q, k, v, scale):
    """f64 softmax(q k^T * scale) v for one head; q [d], k/v [ctx, d]."""
    s = (k @ q) * scale
    s = s - s.max()
    p = np.exp(s)
    return (p @ v) / p.sum()


def attention_inputs(dtype, ctx, hq, hkv, head_dim, pool, seed, num_layers=1, sigma=0.5,
                     outliers=0.0):
    rng = np.random.default_rng(seed)
    npages = (ctx + PAGE - 1) // PAGE
    table = np.zeros(max(npages, 1) + 4, dtype=np.int32)
    table[:npages] = rng.permutation(pool)[:npages]
    shape = (pool, num_layers, hkv, PAGE, head_dim)
    kf = rng.standard_normal(shape) * sigma
    vf = rng.standard_normal(shape) * sigma
    if outliers:
        kf[rng.random(shape) < outliers] *= 8
        vf[rng.random(shape) < outliers] *= 8
    q = bits(rng.standard_normal((hq, head_dim)) * sigma, dtype)
    return q, bits(kf, dtype), bits(vf, dtype), table


def check_attention(orc, dtype, ctx, hq=14, hkv=2, head_dim=64, seed=0, layer=0, num_layers=1,
                    outliers=0.0):
    """Oracle flash_decoding vs f64 textbook attention on the same rounded
    inputs.  The oracle's f32 pipeline adds a few f32 ulps of relative error
    before the single rounding to storage, so the bound is one storage ulp of
    the f64 value plus an f32-level slack."""
    pool = (ctx + PAGE - 1) // PAGE + 7
    q, kp, vp, table = attention_inputs(dtype, ctx, hq, hkv, head_dim, pool, seed, num_layers,
                                        outliers=outliers)
    scale = float(np.float32(1) / np.sqrt(np.float32(head_dim)))
    got = f32(orc.flash_decoding(q, kp, vp, table, layer, hq, hkv, head_dim, ctx - 1, scale,
                                 PAGE, num_layers, dtype), dtype)
    worst = 0.0
    g = hq // hkv
    qf = f32(q, dtype).astype(np.float64)
    for h in range(hq):
        k, v = gather_kv(kp, vp, table, layer, h // g, ctx, dtype)
        want = textbook_attention(qf[h], k, v, scale)
        vmax = np.abs(v).max()
        tol = ulp(want, dtype) * 1.01 + vmax * 2.0 ** -16
        worst = max(worst, float(np.max(np.abs(got[h] - want) / tol)))
    return worst


def check_attention_sdpa(orc, dtype, ctx, hq=14, hkv=2, head_dim=64, seed=1):
    """Oracle vs torch.nn.functional.scaled_dot_product_attention (float64,
    CPU, GQA expanded) -- an independent library implementation."""
    pool = (ctx + PAGE - 1) // PAGE + 3
    q, kp, vp, table = attention_inputs(dtype, ctx, hq, hkv, head_dim, pool, seed)
    scale = float(np.float32(1) / np.sqrt(np.float32(head_dim)))
    got = f32(orc.flash_decoding(q, kp, vp, table, 0, hq, hkv, head_dim, ctx - 1, scale, PAGE, 1,
                                 dtype), dtype)
    g = hq // hkv
    ks, vs = zip(*[gather_kv(kp, vp, table, 0, h, ctx, dtype) for h in range(hkv)])
    K = torch.from_numpy(np.stack(ks)).repeat_interleave(g, 0)[None]
    V = torch.from_numpy(np.stack(vs)).repeat_interleave(g, 0)[None]
    Q = torch.from_numpy(f32(q, dtype).astype(np.float64))[None, :, None, :]
    want = torch.nn.functional.scaled_dot_product_attention(Q, K, V, scale=scale)[0, :, 0].numpy()
    tol = ulp(want, dtype) * 1.01 + np.abs(V.numpy()).max() * 2.0 ** -16
    return float(np.max(np.abs(got - want) / tol))


def check_attention_invariants(orc, dtype, head_dim=64, seed=3):
    """Closed-form special cases:
      ctx == 1           -> output == V[0] exactly
      K == 0             -> output == mean(V) (to one storage ulp)
      q == 0             -> output == mean(V)
      pages permuted together with the table -> bit-identical output
    Returns the number of failed cases."""
    hq, hkv = 4, 2
    fails = 0
    scale = float(np.float32(1) / np.sqrt(np.float32(head_dim)))
    q, kp, vp, table = attention_inputs(dtype, 1, hq, hkv, head_dim, 5, seed)
    out = orc.flash_decoding(q, kp, vp, table, 0, hq, hkv, head_dim, 0, scale, PAGE, 1, dtype)
    for h in range(hq):
        fails += int(not np.array_equal(out[h], vp[table[0], 0, h // 2, 0]))
    ctx = 77
    q, kp, vp, table = attention_inputs(dtype, ctx, hq, hkv, head_dim, 12, seed + 1)
    for mode in ("k0", "q0"):
        kk, qq = kp.copy(), q.copy()
        if mode == "k0":
            kk[:] = 0
        else:
            qq[:] = 0
        out = f32(orc.flash_decoding(qq, kk, vp, table, 0, hq, hkv, head_dim, ctx - 1, scale, PAGE,
                                     1, dtype), dtype)
        for h in range(hq):
            _, v = gather_kv(kk, vp, table, 0, h // 2, ctx, dtype)
            want = v.mean(axis=0)
            tol = ulp(want, dtype) * 1.01 + 1e-7
            fails += int(np.any(np.abs(out[h] - want) > tol))
    # permute physical pages and remap the table
    perm = np.random.default_rng(seed).permutation(kp.shape[0])
    inv = np.argsort(perm)
    kp2, vp2 = kp[perm].copy(), vp[perm].copy()   # new page j holds old page perm[j]
    table2 = inv[table].astype(np.int32)
    a = orc.flash_decoding(q, kp, vp, table, 0, hq, hkv, head_dim, ctx - 1, scale, PAGE, 1, dtype)
    b = orc.flash_decoding(q, kp2, vp2, table2, 0, hq, hkv, head_dim, ctx - 1, scale, PAGE, 1,
                           dtype)
    fails += int(not np.array_equal(a, b))
    return fails


def check_prefill(orc, dtype, lens=(37, 64, 1), start=(0, 5, 130), hq=14, hkv=2, head_dim=64,
                  seed=5):
    """Oracle prefill vs f64 causal attention: each prompt row attends to the
    cache prefix [0, start) (pre-filled) plus prompt rows up to itself, with
    K roped at its position.  RoPE/cache-write are pinned separately, so the
    expected values take the oracle's written pool as the K/V source and
    check the causal structure and the attention itself."""
    rng = np.random.default_rng(seed)
    B = len(lens)
    row = (hq + 2 * hkv) * head_dim
    max_pages = max((s + n + PAGE - 1) // PAGE for s, n in zip(start, lens)) + 1
    pool = B * max_pages + 2
    perm = rng.permutation(pool).astype(np.int32)
    tables = perm[: B * max_pages].reshape(B, max_pages).copy()
    shape = (pool, 1, hkv, PAGE, head_dim)
    kp = bits(rng.standard_normal(shape) * 0.5, dtype)
    vp = bits(rng.standard_normal(shape) * 0.5, dtype)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    qkv = bits(rng.standard_normal((int(cu[-1]), row)) * 0.5, dtype)
    cos, sin = orc.rope_table(1024, head_dim, 1e6)
    scale = float(np.float32(1) / np.sqrt(np.float32(head_dim)))
    qkv2, kp2, vp2 = qkv.copy(), kp.copy(), vp.copy()
    out = f32(orc.prefill(qkv2, None, None, None, cos, sin, kp2, vp2, tables, cu,
                          np.array(start, np.int32), 0, hq, hkv, head_dim, scale, PAGE, 1, dtype),
              dtype)
    worst = 0.0
    g = hq // hkv
    for b in range(B):
        for t in range(lens[b]):
            r = cu[b] + t
            pos = start[b] + t
            qf = f32(qkv2[r, : hq * head_dim].reshape(hq, head_dim), dtype).astype(np.float64)
            for h in range(hq):
                k, v = gather_kv(kp2, vp2, tables[b], 0, h // g, pos + 1, dtype)
                want = textbook_attention(qf[h], k, v, scale)
                tol = ulp(want, dtype) * 1.01 + np.abs(v).max() * 2.0 ** -16
                worst = max(worst, float(np.max(np.abs(out[r, h] - want) / tol)))
            # the prompt's own K/V landed at its position (roped k row, v row)
            page, slot = tables[b][pos // PAGE], pos % PAGE
            kd = hq * head_dim
            kv_dim = hkv * head_dim
            if not np.array_equal(kp2[page, 0, :, slot].reshape(-1), qkv2[r, kd: kd + kv_dim]):
                worst = max(worst, 1e9)
            if not np.array_equal(vp2[page, 0, :, slot].reshape(-1),
                                  qkv2[r, kd + kv_dim: kd + 2 * kv_dim]):
                worst = max(worst, 1e9)
    return worst


# ---------------------------------------------------------------- model-loop ops
def check_rmsnorm(orc, seed=7):
    """Oracle RMSNorm vs the f64 value x / sqrt(mean(x^2) + eps) * w: within
    half a bf16 unit plus the f32 arithmetic's few units of 2^-24.  Short rows
    (8, 16 columns) make a wrong divisor or a dropped eps visible."""
    rng = np.random.default_rng(seed)
    worst = 0.0
    for rows, cols, sigma, eps in [(3, 896, 1.0, 1e-6), (2, 8, 0.5, 1e-6), (4, 16, 3.0, 1e-6),
                                   (2, 64, 1e-3, 1e-6), (1, 4864, 20.0, 1e-5)]:
        x = bits(rng.standard_normal((rows, cols)) * sigma, "bf16")
        w = bits(1 + 0.3 * rng.standard_normal(cols), "bf16")
        got = f32(orc.rmsnorm(x, w, eps), "bf16").astype(np.float64)
        xf = f32(x, "bf16").astype(np.float64)
        want = xf / np.sqrt(np.mean(xf * xf, axis=1, keepdims=True) + np.float32(eps)) * f32(w, "bf16")
        tol = ulp(want, "bf16") * 0.5 + np.abs(want) * 2.0 ** -18 + 1e-30
        worst = max(worst, float(np.max(np.abs(got - want) / tol)))
    return worst


def check_silu_mul(orc, seed=8):
    """gate <- silu(gate) * up vs f64 g / (1 + e^-g) * u (half a bf16 unit plus
    the f32 exp's error); the up half must come back unchanged."""
    rng = np.random.default_rng(seed)
    rows, inter = 5, 512
    gu = bits(rng.standard_normal((rows, 2 * inter)) * 4, "bf16")
    gu[0, :8] = bits(np.array([0.0, -0.0, 20.0, -20.0, 88.0, -88.0, 1e-3, -1e-3]), "bf16")
    got = orc.silu_mul(gu.copy(), inter)
    if not np.array_equal(got[:, inter:], gu[:, inter:]):
        return 1e9
    g = f32(gu[:, :inter], "bf16").astype(np.float64)
    u = f32(gu[:, inter:], "bf16").astype(np.float64)
    want = g / (1 + np.exp(-g)) * u
    tol = ulp(want, "bf16") * 0.5 + np.abs(want) * 2.0 ** -18 + 1e-30
    return float(np.max(np.abs(f32(got[:, :inter], "bf16") - want) / tol))


def argmax_tie_order(v):
    """The reference kernel's greedy index (sampling.cu:16-46, 1024 threads):
    among the largest values above -1e30 (NaN never), the smallest i mod 1024,
    then the smallest i; -1 if none.  Stated from the maxima directly, not by
    simulating threads."""
    v = np.where(np.isnan(v), -np.inf, np.asarray(v, np.float64))
    if v.size == 0 or v.max() <= -1e30:
        return -1
    tied = np.flatnonzero(v == v.max())
    return int(tied[np.lexsort((tied, tied % 1024))][0])


def argmax_cases(rng):
    """Logit rows for the greedy index: random rows, three equal maxima, a NaN
    in front, equal maxima at 600 and 1500 (1500 mod 1024 = 476 < 600, so
    1500 wins), at 1024 and 2048 (thread 0 both: 1024 wins), at 3077 and
    149509 (thread 5 both, the first in a thread's blocks of sixteen loads and
    the second past them: 3077 wins), and a row with nothing above -1e30."""
    out = []
    for n in (1, 7, 1000, 2100, 8200, 151936):
        x = bits(rng.standard_normal(n), "bf16")
        out.append(x)
        if n > 3:
            y = x.copy()
            y[[1, n // 2, n - 1]] = bits(np.array([9.0, 9.0, 9.0]), "bf16")  # ties
            z = y.copy()
            z[0] = 0x7fc0                                                     # NaN first
            out += [y, z]
        if n > 2048:
            w = x.copy()
            w[[600, 1500]] = bits(np.array([9.0, 9.0]), "bf16")
            out.append(w)
            u = x.copy()
            u[[1024, 2048]] = bits(np.array([9.0, 9.0]), "bf16")
            out.append(u)
        if n > 150000:
            v = x.copy()
            v[[5 + 1024 * 3, 5 + 1024 * 146]] = bits(np.array([9.0, 9.0]), "bf16")
            out.append(v)
        out.append(bits(np.full(n, -1e31), "bf16"))
    return out


def check_argmax(orc, seed=9):
    """Greedy index vs argmax_tie_order.  Returns the number of misses."""
    rng = np.random.default_rng(seed)
    return sum(int(orc.argmax(c) != argmax_tie_order(f32(c, "bf16"))) for c in argmax_cases(rng))


# ---------------------------------------------------------------- top-k / top-p sampling
def _bitrev5(x):
    x = np.asarray(x, dtype=np.int64)
    r = np.zeros_like(x)
    for b in range(5):
        r |= ((x >> b) & 1) << (4 - b)
    return r


def topk_closed_form(logits_bits, k_per_block):
    """Candidates of top_k_filter in closed form.  In each of the 32 partitions
    the valid items (value > -1e30, not NaN) are ordered by value, descending;
    equal values are ordered the way the reference's trees resolve them: a
    shfl_down max tree that keeps the lower slot's pair on ties makes lane bit 0
    the most significant tie bit, then bit 1, ..., i.e. the smallest
    bit-reversed lane wins, first over the 8 warps (warp = (i % 256) // 32),
    then over the lanes ((i % 256) % 32), and a thread's own strided scan keeps
    its smallest i.  The first k_per_block are taken; missing ones are
    (start - 1, -1e30)."""
    v = f32(logits_bits, "bf16").astype(np.float32)
    n_all = v.size
    keys, vals = [], []
    for p in range(32):
        start, end = p * n_all // 32, (p + 1) * n_all // 32
        x = v[start:end]
        i = np.arange(end - start)
        ok = ~np.isnan(x) & (x > np.float32(-1e30))
        t = i % 256
        order = np.lexsort((i // 256, _bitrev5(t % 32), _bitrev5(t // 32), -x.astype(np.float64)))
        order = order[ok[order]][:k_per_block]
        kk = list(start + order) + [start - 1] * (k_per_block - order.size)
        vv = list(x[order]) + [np.float32(-1e30)] * (k_per_block - order.size)
        keys += kk
        vals += vv
    return np.array(keys, np.int32), np.array(vals, np.float32)


def sampling_logits(n, seed, levels=None, specials=True):
    """bf16 logits with many equal values (levels > 0 quantises them) and, with
    specials, NaN, -inf, values <= -1e30 and a partition with few valid items."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(n) * 3.0
    if levels:
        x = np.round(x * levels) / levels
    b = bits(x, "bf16")
    if specials and n >= 64:
        b[rng.integers(0, n, max(1, n // 500))] = 0x7fc0          # NaN
        b[rng.integers(0, n, max(1, n // 500))] = 0xff80          # -inf
        b[rng.integers(0, n, max(1, n // 500))] = bits(np.array([-1e30]), "bf16")[0]
        b[rng.integers(0, n, max(1, n // 500))] = bits(np.array([-3e35]), "bf16")[0]
        b[rng.integers(0, n, max(2, n // 200))] = 0x8000                 # -0 ties with +0
        b[rng.integers(0, n, max(2, n // 200))] = 0x0000
        e = n * 3 // 32                                            # partition 2: 5 valid items
        b[2 * n // 32:e] = 0xff80
        b[2 * n // 32:e][:: max(1, (e - 2 * n // 32) // 5)][:5] = bits(np.arange(5.0), "bf16")
    return b


def signed_zero_logits(n, seed):
    """Negative logits with scattered +0 and -0: the zeros are the largest
    values and tie with each other."""
    rng = np.random.default_rng(seed)
    b = bits(-np.abs(rng.standard_normal(n)) - 0.01, "bf16")
    b[rng.integers(0, n, n // 40)] = 0x8000
    b[rng.integers(0, n, n // 40)] = 0x0000
    return b


def sampling_cases(seed):
    """(logits bits, k_per_block) cases of the filter checks."""
    cases = [(sampling_logits(n, seed + n, levels), kpb)
             for n, kpb, levels in ((151936, 32, 4), (151936, 4, None), (1000, 32, 2),
                                    (40000, 8, 1), (33, 1, None), (8192, 16, 8))]
    cases.append((signed_zero_logits(12000, seed), 32))
    # every logit equal: the order is the tie order alone, and with 32 per
    # partition more than 1024 items of a partition tie with the 32nd
    cases.append((bits(np.ones(32 * 4748), "bf16"), 32))
    # the largest values of every partition crowded into the items whose
    # partition-local index is below 64 modulo 1024
    rng = np.random.default_rng(seed + 1)
    x = rng.standard_normal(32 * 4748) - 5.0
    loc = np.arange(32 * 4748) % 4748
    x[loc % 1024 < 64] += 15.0
    cases.append((bits(x, "bf16"), 32))
    return cases


def check_topk_filter(orc, seed=21):
    """Oracle candidates vs the closed form (keys and value bits exact), on
    vocabularies that are and are not multiples of 32, with ties.  Returns the
    number of mismatching candidates."""
    fails = 0
    for b, kpb in sampling_cases(seed):
        k1, v1 = orc.topk_filter(b, kpb)
        k2, v2 = topk_closed_form(b, kpb)
        fails += int(np.sum((k1 != k2) | (v1.view(np.uint32) != v2.view(np.uint32))))
    return fails


def _bitonic_recursive(keys, vals):
    """Batcher's bitonic sort, recursive form: a block of size m at offset lo
    sorts descending when (lo // m) is even (so every block at the top is
    descending, its first half descending and its second ascending), then
    merges by compare-exchanges at distance m/2, m/4, ... that swap only on a
    strict inequality."""
    keys, vals = list(keys), list(vals)

    def merge(lo, m, down):
        if m < 2:
            return
        h = m // 2
        for i in range(lo, lo + h):
            if (vals[i] < vals[i + h]) if down else (vals[i] > vals[i + h]):
                keys[i], keys[i + h] = keys[i + h], keys[i]
                vals[i], vals[i + h] = vals[i + h], vals[i]
        merge(lo, h, down)
        merge(lo + h, h, down)

    def sort(lo, m):
        if m < 2:
            return
        sort(lo, m // 2)
        sort(lo + m // 2, m // 2)
        merge(lo, m, (lo // m) % 2 == 0)

    sort(0, len(vals))
    return np.array(keys, np.int32), np.array(vals, np.float32)


def check_bitonic(orc, seed=22):
    """Oracle network vs the recursive form (exact, ties included), and the
    output is a permutation sorted by value, descending.  Returns misses."""
    rng = np.random.default_rng(seed)
    fails = 0
    for n in (32, 64, 256, 1024):
        for levels in (None, 2, 0.25):
            x = rng.standard_normal(n) * 3
            if levels:
                x = np.round(x * levels) / levels
            vals = x.astype(np.float32)
            keys = rng.permutation(100000)[:n].astype(np.int32)
            k1, v1 = orc.bitonic_desc(keys, vals)
            k2, v2 = _bitonic_recursive(keys, vals)
            fails += int(np.sum(k1 != k2) + np.sum(v1 != v2))
            fails += int(np.any(np.diff(v1) > 0))
            fails += int(not np.array_equal(np.sort(k1), np.sort(keys)))
    return fails


def top_p_closed_form(vals, top_p, rand_val):
    """Position picked from sorted values in f64, and the smallest distance of
    top_p and of the target to an interval end (ties within it are not
    decided by this form)."""
    v = np.asarray(vals, np.float64)
    e = np.exp(v - v[0])
    prob = e / e.sum()
    cdf = np.cumsum(prob)
    prev = cdf - prob
    hit = np.nonzero((prev < top_p) & (cdf >= top_p))[0]
    cutoff = cdf[hit[0]] if hit.size else 1.0
    target = rand_val * cutoff
    win = np.nonzero((cdf >= target) & (prev < target))[0]
    margin = min(np.min(np.abs(cdf - top_p)), np.min(np.abs(cdf - target)))
    return (int(win[0]) if win.size else -1), margin


def check_top_p(orc, seed=23):
    """The sample step vs the f64 closed form where no interval end lies
    within 1e-5 of top_p or the target, plus exact cases: a single
    dominating candidate, an exact top_p boundary, rand 0 (no winner).
    Returns misses."""
    rng = np.random.default_rng(seed)
    fails = 0
    decided = 0
    for n in (32, 128, 1024):
        for _ in range(60):
            vals = np.sort(rng.standard_normal(n).astype(np.float32) * rng.uniform(0.5, 4))[::-1]
            vals = np.ascontiguousarray(vals)
            top_p, r = float(rng.uniform(0.05, 1.0)), float(rng.uniform(0, 1))
            want, margin = top_p_closed_form(vals, top_p, r)
            if margin < 1e-5:
                continue
            decided += 1
            fails += int(orc.top_p_pick(vals, top_p, r)[0] != want)
    fails += int(decided < 150)
    # two equal leaders, the rest negligible: prob (0.5, 0.5, 0 ...); top_p = 0.5
    # is the first interval's end exactly, so the cutoff is 0.5 and any rand
    # picks position 0 (a strict cutoff test would pick position 1 for rand 0.75)
    vals = np.array([5.0, 5.0] + [-1e30] * 30, np.float32)
    fails += int(orc.top_p_pick(vals, 0.5, 0.75)[0] != 0)
    fails += int(orc.top_p_pick(vals, 0.9, 0.75)[0] != 1)
    fails += int(orc.top_p_pick(vals, 0.9, 0.0)[0] != -1)          # rand 0: no winner
    big = np.array([40.0] + [0.0] * 31, np.float32)                 # one candidate holds ~1
    fails += int(orc.top_p_pick(big, 0.3, 0.999)[0] != 0)
    return fails


# ---------------------------------------------------------------- model composition
def tiny_qwen_weights(cfg, seed, std=0.15):
    """Random weights in the fused layout (bf16 bits), larger than an HF init
    so attention is far from uniform and every term moves the logits."""
    rng = np.random.default_rng(seed)
    H, I, V = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
    qkv_dim = H + 2 * cfg.num_key_value_heads * cfg.head_dim
    nb = lambda *s, mean=0.0: bits(mean + std * rng.standard_normal(s), "bf16")  # noqa: E731
    w = {"embed_tokens": bits(rng.standard_normal((V, H)), "bf16"), "final_norm": nb(H, mean=1.0),
         "layers": []}
    for _ in range(cfg.num_hidden_layers):
        w["layers"].append({"input_layernorm": nb(H, mean=1.0), "qkv_proj": nb(qkv_dim, H),
                            "qkv_bias": nb(qkv_dim), "o_proj": nb(H, H),
                            "post_attention_layernorm": nb(H, mean=1.0),
                            "gate_up_proj": nb(2 * I, H), "down_proj": nb(H, I)})
    return w


def qwen2_f64(cfg, w, ids):
    """Textbook Qwen2 decoder in float64 over the whole sequence (causal
    attention, rotate-half RoPE with theta_i = pos / base^(2i/d), GQA, SwiGLU,
    pre-norm residuals, tied lm_head); returns the last row's logits."""
    F = lambda b: f32(b, "bf16").astype(np.float64)  # noqa: E731
    H, d = cfg.hidden_size, cfg.head_dim
    hq, hkv, I = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.intermediate_size
    S = len(ids)
    eps = cfg.rms_norm_eps

    def norm(x, g):
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * F(g)

    pos = np.arange(S, dtype=np.float64)[:, None]
    inv = 1.0 / np.power(cfg.rope_theta, np.arange(d // 2) * 2.0 / d)
    c, s = np.cos(pos * inv)[:, None, :], np.sin(pos * inv)[:, None, :]

    def rope(x):  # [S, heads, d]
        a, b = x[..., : d // 2], x[..., d // 2:]
        return np.concatenate([a * c - b * s, a * s + b * c], axis=-1)

    h = F(w["embed_tokens"])[np.asarray(ids)]
    mask = np.triu(np.full((S, S), -np.inf), 1)
    for L in w["layers"]:
        x = norm(h, L["input_layernorm"])
        qkv = x @ F(L["qkv_proj"]).T + F(L["qkv_bias"])
        q = rope(qkv[:, :H].reshape(S, hq, d))
        k = rope(qkv[:, H: H + hkv * d].reshape(S, hkv, d))
        v = qkv[:, H + hkv * d:].reshape(S, hkv, d)
        att = np.empty((S, hq, d))
        for hh in range(hq):
            kv = hh // (hq // hkv)
            sc = q[:, hh] @ k[:, kv].T / np.sqrt(d) + mask
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            att[:, hh] = (p / p.sum(axis=1, keepdims=True)) @ v[:, kv]
        h = h + att.reshape(S, H) @ F(L["o_proj"]).T
        x = norm(h, L["post_attention_layernorm"])
        gu = x @ F(L["gate_up_proj"]).T
        g, u = gu[:, :I], gu[:, I:]
        h = h + (g / (1 + np.exp(-g)) * u) @ F(L["down_proj"]).T
    return norm(h[-1:], w["final_norm"])[0] @ F(w["embed_tokens"]).T


def check_oracle_model(orc, seed=11):
    """The oracle's Qwen2 loop (bf16 at the reference's rounding points) vs
    the f64 textbook decoder on a tiny config: prefill of 6 tokens then 4
    decode steps, rms logit error within 4% of the rms logit at every step.
    bf16 rounding at the reference's points gives about 1.5%; a dropped q/k or
    v bias, interleaved instead of rotate-half RoPE, a wrong GQA map or
    softmax scale, no causal mask, a swapped norm weight, silu applied to up or
    no final norm each give 22% or more.  Returns the worst error relative to
    that tolerance."""
    from oracle.model import OracleQwen2
    from types import SimpleNamespace
    cfg = SimpleNamespace(vocab_size=300, hidden_size=128, num_hidden_layers=2, num_attention_heads=4,
                          num_key_value_heads=2, intermediate_size=256, rms_norm_eps=1e-6,
                          rope_theta=10000.0, head_dim=32)
    w = tiny_qwen_weights(cfg, seed)
    m = OracleQwen2(cfg, w, max_positions=64, num_blocks=8)
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, cfg.vocab_size, 10).tolist()
    worst = 0.0
    for step in range(5):
        if step == 0:
            m.forward(ids[:6], 0)
            seq = ids[:6]
        else:
            m.forward([ids[5 + step]], 5 + step)
            seq = ids[: 6 + step]
        got = f32(m.logits(), "bf16").astype(np.float64)
        want = qwen2_f64(cfg, w, seq)
        tol = 0.04 * np.sqrt(np.mean(want * want))
        worst = max(worst, float(np.sqrt(np.mean((got - want) ** 2)) / tol))
    return worst
