"""Needle inputs for the prefill path: every key of a (sequence, kv head) is
zero except one token t*, whose key is the common query direction.  Every
prompt row's q (all heads) is 16 on the four lowest-frequency rotation pairs
(dims d/2-4 .. d/2-1, zero on their partners) before RoPE; the needle's key
is the same vector, roped at t* (a cached prefix slot written here, or a
prompt row's k that the append kernel ropes).  After RoPE the needle's score
for a row at position p is 256 * sum_j cos((p - t*) theta_j) over those four
pairs: at least 1023.9 for |p - t*| < 4096, since theta_j <= 1e6^(-(d-8)/d)
keeps every angle below 0.03 rad.  Scaled, that is 128 (head_dim 64) or 90.5
(128); every other score is exactly 0.  So every row whose causal context
holds t* (p >= t*) outputs V[t*] bit for bit in every q-head of the unit, and
every row before it (p < t*) outputs the mean of the V rows it sees, which is
not V[t*].  t* sits at the first and last token of pages (16), 32-row tiles
(counted from the prompt's first row), 64-token blocks and 128-token super
blocks (counted from position 0), at the first prompt row and the last
cached one, and on the diagonal (t* is then a prompt row's own position);
unused slots and table entries hold NaN, so a read outside a row's causal
range shows up.  Shared by the GPU needle test and its CPU pin against the
oracle.  The semantics are the reference's per-token loop
(src/models.rs:485-550) and its causal addressing (src/kernels/attention.cu:80-87)."""
import numpy as np

from lucciola_rs_amd import workloads as wl

PAGE = 16

# (prompt rows, cached prefix) per sequence: one-row prompts, prompts ending
# on and past a 32-row tile, prefixes on and off page and block edges
SEQS = [(1, 0), (33, 5), (64, 16), (97, 31), (128, 64), (200, 100), (31, 130), (300, 7)]


def candidates(start: int, rows: int):
    """Needle positions for a sequence: page, block and super-block edges from
    position 0, tile edges from the prompt's first row, the first prompt row,
    the last cached token and the last row (all inside the context)."""
    ctx = start + rows
    cand = {0, ctx - 1, start, start - 1}
    for unit in (16, 64, 128):
        for k in range(1, ctx // unit + 1):
            cand |= {k * unit - 1, k * unit}
    for k in range(1, rows // 32 + 1):
        cand |= {start + 32 * k - 1, start + 32 * k}
    return sorted(p for p in cand if 0 <= p < ctx)


def needle_prefill_inputs(cfg, seed, cos, sin, seqs=SEQS):
    """Host prefill inputs with one needle per (sequence, kv head); returns
    them, the needle positions [B, Hkv] and the V row each needle selects
    [B, Hkv, d] (bits)."""
    rows = np.array([r for r, _ in seqs])
    starts = np.array([s for _, s in seqs])
    h = wl.host_prefill_inputs(cfg, seed=seed, rows=rows, starts=starts, poison=True)
    d, hq, hkv = cfg.head_dim, cfg.hq, cfg.hkv
    half = d // 2
    k_pool = h.k_pool.copy()
    finite = ~np.isnan(wl.bits_to_tensor(k_pool, cfg.dtype).float().numpy())
    k_pool[finite] = 0  # every cached key zero (NaN poison stays)
    qv = np.zeros(d, np.float64)
    qv[half - 4: half] = 16.0
    q_bits = wl.to_bits(qv.astype(np.float32), cfg.dtype)
    qkv = h.qkv.copy()
    qkv[:, : hq * d] = np.tile(q_bits, hq)
    qkv[:, hq * d:(hq + hkv) * d] = 0  # every prompt row's k zero
    needles = np.zeros((len(seqs), hkv), np.int64)
    vsel = np.zeros((len(seqs), hkv, d), np.uint16)
    rng = np.random.default_rng(seed + 1000)
    for b, (n, s) in enumerate(seqs):
        cands = candidates(s, n)
        for kv in range(hkv):
            t = int(cands[rng.integers(len(cands))])
            needles[b, kv] = t
            if t < s:  # a cached key: qv roped at t (pairs i, i + d/2), rounded
                c, sn = cos[t].astype(np.float64), sin[t].astype(np.float64)
                key = np.concatenate([qv[:half] * c - qv[half:] * sn, qv[:half] * sn + qv[half:] * c])
                slot = (h.tables[b, t // PAGE], 0, kv, t % PAGE)
                k_pool[slot] = wl.to_bits(key.astype(np.float32), cfg.dtype)
                vsel[b, kv] = h.v_pool[slot]
            else:  # a prompt row's k: roped at t by the append step
                r = int(h.cu_seqlens[b]) + t - s
                qkv[r, (hq + kv) * d:(hq + kv + 1) * d] = q_bits
                vsel[b, kv] = qkv[r, (hq + hkv + kv) * d:(hq + hkv + kv + 1) * d]
    hn = wl.HostPrefill(cfg, 1, h.cu_seqlens, h.start_pos, h.tables, qkv, k_pool, h.v_pool)
    return hn, needles, vsel


def needle_mismatches(h, needles, vsel, out_bits):
    """(rows at or past the needle whose output differs from V[t*], rows
    before it whose output equals V[t*] in every dim of some head) over every
    (sequence, kv head); out_bits [total_rows, Hq, d]."""
    cfg = h.cfg
    G = cfg.hq // cfg.hkv
    late, early = 0, 0
    for b in range(len(needles)):
        r0, r1 = int(h.cu_seqlens[b]), int(h.cu_seqlens[b + 1])
        pos = int(h.start_pos[b]) + np.arange(r1 - r0)
        for kv in range(cfg.hkv):
            o = out_bits[r0:r1, kv * G:(kv + 1) * G]           # [rows, G, d]
            same = np.all(o == vsel[b, kv][None, None, :], axis=2)  # [rows, G]
            sees = pos >= needles[b, kv]
            late += int(np.sum(~same[sees]))
            early += int(np.sum(same[~sees]))
    return late, early
