"""The C-ABI library loads and exports every declared entry point; host-side
argument checks reject bad calls before any GPU work (CPU only)."""
import ctypes
import glob
import os
import re

import pytest
import numpy as np
import torch

from lucciola_rs_amd import library

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(luc_\w+)\s*\(", text))
    return sorted(names)


def test_header_declares_entry_points():
    names = declared_functions()
    assert "luc_paged_decode" in names and "luc_rope_append" in names
    assert len(names) >= 10


def test_library_exports_every_declared_symbol():
    cdll = library.load_cdll()
    missing = [n for n in declared_functions() if not hasattr(cdll, n)]
    assert not missing, missing
    # and the ctypes signature table covers them all
    assert set(declared_functions()) <= set(library.SIGNATURES)


def test_code_objects_built_for_gfx950():
    for name in ("rope_append", "paged_decode", "paged_decode_w8"):
        path = os.path.join(library.lib_dir(), name + ".hsaco")
        data = open(path, "rb").read()
        assert data[:4] == b"\x7fELF"
        assert b"gfx950" in data


def test_abi_version_and_error_string():
    cdll = library.load_cdll()
    assert cdll.luc_abi_version() == 4
    rc = cdll.luc_paged_decode(None, None, 0, None, 0, None, 0, None, None, None, 0, 1, None, 1,
                               1, 0, 1, 14, 2, 64, 16, 0.125, 0, None, 0)
    assert rc == -1
    assert b"null context" in cdll.luc_last_error()


class FakeCtx:
    """Host checks run before the context is dereferenced for any GPU call;
    a non-null dummy handle reaches them."""


@pytest.fixture
def cdll():
    return library.load_cdll()


def _decode(cdll, **kw):
    args = dict(ctx=ctypes.c_void_p(1), stream=None, dtype=0, out=ctypes.c_void_p(16),
                out_stride=14 * 64, q=ctypes.c_void_p(16), q_stride=14 * 64,
                k_pool=ctypes.c_void_p(256), v_pool=ctypes.c_void_p(512),
                tables=ctypes.c_void_p(16), table_stride=256, num_blocks=16384,
                positions=ctypes.c_void_p(16), batch=32, max_ctx=4096, layer=0, num_layers=24,
                hq=14, hkv=2, head_dim=64, block_size=16, scale=0.125, split=0, ws=None,
                ws_bytes=0)
    args.update(kw)
    rc = cdll.luc_paged_decode(*args.values())
    return rc, cdll.luc_last_error().decode()


def test_decode_argument_checks(cdll):
    assert _decode(cdll, head_dim=96)[0] == -2             # kernels.rs:37-46
    assert _decode(cdll, block_size=32)[0] == -2           # kv_cache.rs:35
    assert _decode(cdll, hq=18, hkv=2)[0] == -2            # group 9 > 8
    assert _decode(cdll, hq=15, hkv=2)[0] == -1            # not a multiple
    assert _decode(cdll, k_pool=ctypes.c_void_p(8))[0] == -1   # misaligned pool
    assert _decode(cdll, layer=24)[0] == -1
    assert _decode(cdll, table_stride=100)[0] == -1        # 100 pages < 4096 tokens
    assert _decode(cdll, q_stride=100)[0] == -1
    assert _decode(cdll, dtype=7)[0] == -1
    assert _decode(cdll, positions=None)[0] == -1
    assert _decode(cdll, batch=0)[0] == 0                  # empty batch: no-op
    assert _decode(cdll, max_ctx=0)[0] == -1
    assert _decode(cdll, num_blocks=0)[0] == -1           # a pool of no pages
    rc, msg = _decode(cdll, num_blocks=-3)
    assert rc == -1 and "num_blocks" in msg


def test_workspace_size_policy(cdll):
    ws = cdll.luc_paged_decode_workspace_size

    def expect(batch, hq, hkv, d, splits):
        # 256-byte aligned sections: 65536 int32 arrival counters (a fixed
        # size, so one workspace serves calls of any sizes), (max, sum) in f32
        # per (sequence, q-head, split), o[d] in f32 per (sequence, q-head, split)
        a256 = lambda n: -(-n // 256) * 256  # noqa: E731
        return 65536 * 4 + a256(batch * hq * splits * 8) + a256(batch * hq * splits * d * 4)

    # one split per sequence -> no workspace
    assert ws(32, 14, 2, 64, 100, 0) == 0
    assert ws(2, 14, 2, 64, 1000, 256) == expect(2, 14, 2, 64, 4)
    assert ws(100, 28, 4, 128, 1000, 128) == expect(100, 28, 4, 128, 8)
    # at most 256 splits per sequence: the split grows with the context
    assert ws(1, 4, 1, 64, 64 * 1024, 64) == expect(1, 4, 1, 64, 256)
    # rounding of the requested split to 4 tiles (4 x 64 tokens at d=64,
    # 4 x 32 at d=128)
    assert ws(2, 14, 2, 64, 1000, 100) == ws(2, 14, 2, 64, 1000, 256)
    assert ws(2, 14, 2, 64, 1000, 257) == expect(2, 14, 2, 64, 2)
    assert ws(2, 14, 2, 128, 1000, 90) == ws(2, 14, 2, 128, 1000, 128)
    assert ws(1, 4, 1, 96, 1000, 0) == 0
    # the automatic split keeps about 2048 tiles per round: the batch32_mixed
    # shape (mean context about half of 4096) gets one tile per wave, in the
    # 8-wave single-tile kernel: 8 tiles of 64 tokens per split
    assert ws(32, 14, 2, 64, 4096, 0) == expect(32, 14, 2, 64, 8)
    # ... and longer batches get longer splits, planned for half as many
    # tiles once they need the two-tile kernels (two workgroups per CU):
    # batch64_long (64 x 4 units, 16384 tokens) -> 2048-token splits, several
    # rounds of 4-wave workgroups
    assert ws(64, 28, 4, 128, 16384, 0) == expect(64, 28, 4, 128, 16384 // 2048)
    # a plan of one round of 4-wave workgroups (8 x 2 units of 32 1024-token
    # splits) takes twice the split on 8-wave ones if those fit one round
    # (16 x 16 <= 256 workgroups): batch8_32k -> 2048-token splits
    assert ws(8, 12, 2, 128, 32768, 0) == expect(8, 12, 2, 128, 32768 // 2048)
    # ... and keeps its split where they would not: 24 units of 21 768-token
    # splits (504 4-wave workgroups) would take 24 x 11 > 256 at 1536 tokens
    assert ws(12, 12, 2, 128, 16000, 0) == expect(12, 12, 2, 128, -(-16000 // 768))
    # a split holds at most 128 pages: longer contexts than 256 x 2048 tokens
    # are not supported
    assert ws(1, 4, 1, 64, 256 * 2048, 0) > 0
    assert ws(1, 4, 1, 64, 256 * 2048 + 1, 0) == 0


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("scale", [0.0, 2.0, 4.0])
def test_rope_table_entry_point_matches_oracle(orc, cdll, head_dim, scale):
    """luc_rope_table (RopeCache::new, src/layers/rope.rs:21-29) over the whole
    Qwen2.5 position range: bit-equal to the oracle's table, and within the
    f64 closed form's f32 bound (theta = (pos / scale) / base^(2i/d))."""
    import pins
    max_pos = 32768
    cos = torch.empty(max_pos, head_dim // 2)
    sin = torch.empty(max_pos, head_dim // 2)
    assert cdll.luc_rope_table(ctypes.c_void_p(cos.data_ptr()), ctypes.c_void_p(sin.data_ptr()),
                               max_pos, head_dim, 1e6, scale) == 0
    oc, os_ = orc.rope_table(max_pos, head_dim, 1e6, scale or None)
    assert torch.equal(cos, torch.from_numpy(oc)) and torch.equal(sin, torch.from_numpy(os_))
    pos = np.arange(max_pos, dtype=np.float64)[:, None]
    i = np.arange(head_dim // 2, dtype=np.float64)[None, :]
    theta = (pos / (scale or 1.0)) / np.power(1e6, 2 * i / head_dim)
    tol = np.abs(theta) * 2.0 ** -21 + 2.0 ** -23
    err = np.maximum(np.abs(cos.numpy() - np.cos(theta)), np.abs(sin.numpy() - np.sin(theta)))
    assert float(np.max(err / tol)) <= 1.0
    assert cdll.luc_rope_table(None, None, 512, head_dim, 1e6, 0.0) == -1


def test_init_without_device_fails_cleanly(cdll):
    if torch.cuda.is_available():
        pytest.skip("a device is present")
    ctx = ctypes.c_void_p()
    rc = cdll.luc_init(0, None, ctypes.byref(ctx))
    assert rc in (-1, -4) and not ctx.value


def test_decode_step_argument_checks(cdll):
    def call(**kw):
        args = dict(ctx=ctypes.c_void_p(1), stream=None, dtype=1, qkv=ctypes.c_void_p(16),
                    qkv_stride=18 * 64, qb=None, kb=None, vb=None, cos=ctypes.c_void_p(16),
                    sin=ctypes.c_void_p(16), k_pool=ctypes.c_void_p(256),
                    v_pool=ctypes.c_void_p(512), tables=ctypes.c_void_p(16), table_stride=256,
                    num_blocks=16384, positions=ctypes.c_void_p(16), batch=32, max_ctx=4096, layer=0,
                    num_layers=24, hq=14, hkv=2, head_dim=64, block_size=16, scale=0.125,
                    split=0, out=ctypes.c_void_p(16), out_stride=14 * 64, ws=None, ws_bytes=0)
        args.update(kw)
        return cdll.luc_decode_step(*args.values())
    assert call(qkv_stride=14 * 64) == -1      # a qkv row holds q, k and v
    assert call(num_blocks=0) == -1
    assert call(cos=None) == -1
    assert call(head_dim=80) == -2
    assert call(ws=None, ws_bytes=0) == -5     # split-K needs the workspace
    assert call(batch=0) == 0
    need = cdll.luc_paged_decode_workspace_size(32, 14, 2, 64, 4096, 0)
    assert need > 0
    assert call(ws=ctypes.c_void_p(4096 + 8), ws_bytes=need) == -1   # alignment
    assert call(ws=ctypes.c_void_p(4096), ws_bytes=need - 4) == -5   # too small


def test_gemv_argument_checks(cdll):
    """The one-row products reject on the host, before touching the context:
    dtype, k outside [8, 8192] or not a multiple of 8, negative rows, null or
    misaligned operands, a null norm weight; no rows is a no-op."""
    p = ctypes.c_void_p
    def gemv(**kw):
        args = dict(ctx=p(1), stream=None, dtype=0, y=p(256), x=p(256), w=p(512), res=None,
                    n=896, k=896)
        args.update(kw)
        return cdll.luc_gemv(*args.values())
    assert gemv(dtype=1) == -2
    for k in (0, 12, 8200):
        assert gemv(k=k) == -2
    assert gemv(n=-1) == -1
    assert gemv(x=None) == -1
    assert gemv(x=p(258)) == -1               # 16-byte loads of x
    assert gemv(w=p(520)) == -1               # and of w
    assert gemv(n=0) == 0
    def norm_gemv(**kw):
        args = dict(ctx=p(1), stream=None, dtype=0, y=p(256), x=p(256), nw=p(768), eps=1e-6,
                    w=p(512), res=None, n=896, k=896)
        args.update(kw)
        return cdll.luc_rmsnorm_gemv(*args.values())
    assert norm_gemv(nw=None) == -1
    assert norm_gemv(nw=p(776)) == -1
    assert norm_gemv(k=900) == -2
    assert norm_gemv(n=0) == 0
    def gate_up(**kw):
        args = dict(ctx=p(1), stream=None, dtype=0, act=p(256), x=p(256), nw=None, eps=1e-6,
                    w=p(512), inter=4864, k=896)
        args.update(kw)
        return cdll.luc_gate_up_silu(*args.values())
    assert gate_up(dtype=1) == -2
    assert gate_up(k=8208) == -2
    assert gate_up(w=None) == -1
    assert gate_up(inter=0) == 0
    assert gemv(ctx=None) == norm_gemv(ctx=None) == gate_up(ctx=None) == -1


def test_prefill_argument_checks(cdll):
    """luc_paged_prefill rejects bad arguments on the host (no GPU call): the
    alignment its vector loads need, row strides, head sizes, missing arrays
    and a table too short for max_ctx; an empty batch is a no-op."""
    def call(**kw):
        args = dict(ctx=ctypes.c_void_p(1), stream=None, dtype=0, qkv=ctypes.c_void_p(256),
                    qkv_stride=18 * 64, qb=None, kb=None, vb=None, cos=ctypes.c_void_p(16),
                    sin=ctypes.c_void_p(16), k_pool=ctypes.c_void_p(256),
                    v_pool=ctypes.c_void_p(512), tables=ctypes.c_void_p(16), table_stride=129,
                    num_blocks=512, cu=ctypes.c_void_p(16), start=ctypes.c_void_p(16), batch=4,
                    total=8192,
                    max_ctx=2048, layer=0, num_layers=24, hq=14, hkv=2, head_dim=64,
                    block_size=16, scale=0.125, out=ctypes.c_void_p(256), out_stride=14 * 64)
        args.update(kw)
        return cdll.luc_paged_prefill(*args.values())
    assert call(qkv_stride=14 * 64) == -1                 # a qkv row holds q, k and v
    assert call(qkv=ctypes.c_void_p(264)) == -1           # q rows are read as 16-byte vectors
    assert call(qkv_stride=18 * 64 + 4) == -1
    assert call(out=ctypes.c_void_p(260)) == -1           # outputs written as 8-byte vectors
    assert call(out_stride=14 * 64 + 2) == -1
    assert call(cu=None) == -1 and call(start=None) == -1 and call(cos=None) == -1
    assert call(table_stride=127) == -1                   # 127 pages < 2048 tokens
    assert call(num_blocks=0) == -1
    assert call(head_dim=80) == -2
    assert call(hq=18) == -2                              # group 9 > 8
    assert call(hq=15) == -1                              # not a multiple of hkv
    assert call(block_size=32) == -2
    assert call(max_ctx=0) == -1
    assert call(batch=0) == 0 and call(total=0) == 0


def test_sort_and_sample_argument_checks(cdll):
    """luc_sort_and_sample rejects on the host: top_k outside the built
    candidate sizes (the reference's "Unsupported candidate size"), bf16 only,
    a vocabulary the 32 partitions cannot cover, a short or misaligned
    sort buffer and null pointers."""
    def call(**kw):
        args = dict(ctx=ctypes.c_void_p(1), stream=None, dtype=0, logits=ctypes.c_void_p(256),
                    vocab=151936, top_p=0.9, top_k=1024, rand=0.5, buf=ctypes.c_void_p(4096),
                    buf_bytes=8192, out=ctypes.c_void_p(64))
        args.update(kw)
        return cdll.luc_sort_and_sample(*args.values())
    for k in (0, 16, 48, 2048):
        assert call(top_k=k) == -2
        assert b"Unsupported candidate size" in cdll.luc_last_error()
    assert call(dtype=1) == -2
    assert call(vocab=31) == -1 and call(vocab=32 * 16384 + 1) == -1
    assert call(buf_bytes=8191) == -5
    assert call(top_k=32, buf_bytes=255) == -5
    assert call(buf=ctypes.c_void_p(4100)) == -1
    assert call(logits=None) == -1 and call(buf=None) == -1 and call(out=None) == -1
    assert call(ctx=None) == -1


def test_sampler_top_k_rule():
    """Sampler::new's normalisation (src/sampler.rs:19-23)."""
    from lucciola_rs_amd.sampler import normalize_top_k
    assert [normalize_top_k(k) for k in (0, 1, 32, 33, 50, 64, 100, 1000, 1024, 5000)] == \
        [1024, 32, 32, 64, 64, 64, 128, 1024, 1024, 1024]
