"""CPU oracle for the paged-attention path (test infrastructure only).

`oracle/luc_oracle.c` restates the reference's rope / cache-write / decode
attention (src/kernels/rope.cu, src/kernels/kv_cache.cu,
src/kernels/attention.cu, src/layers/rope.rs) on the CPU.  This module binds it
with ctypes.  Only tests, the smoke check and the benchmark's CPU-baseline leg
use it; the product never does.

Storage arrays are numpy uint16 bit patterns (bf16 or fp16), tables int32,
RoPE tables float32.  Build with `make -C oracle`.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

DTYPES = {"bf16": 0, "f16": 1}
_HERE = os.path.dirname(os.path.abspath(__file__))
# LUC_ORACLE_LIB: another build of the same source (the CPU sanitizer build)
LIB_PATH = os.environ.get("LUC_ORACLE_LIB") or os.path.join(_HERE, "libluc_oracle.so")

_u16p = ctypes.POINTER(ctypes.c_uint16)
_i32p = ctypes.POINTER(ctypes.c_int32)
_f32p = ctypes.POINTER(ctypes.c_float)
_i64 = ctypes.c_int64
_int = ctypes.c_int
_flt = ctypes.c_float


def _ptr(arr, kind):
    if arr is None:
        return None
    want = {"u16": np.uint16, "i32": np.int32, "f32": np.float32}[kind]
    if arr.dtype != want:
        raise TypeError(f"expected {want}, got {arr.dtype}")
    if not arr.flags["C_CONTIGUOUS"]:
        raise ValueError("array must be C-contiguous")
    ctype = {"u16": _u16p, "i32": _i32p, "f32": _f32p}[kind]
    return arr.ctypes.data_as(ctype)


def _dt(dtype):
    if isinstance(dtype, int):
        return dtype
    return DTYPES[dtype]


class Oracle:
    """ctypes binding of libluc_oracle.so."""

    def __init__(self, path: str | None = None):
        path = path or LIB_PATH
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        self.lib = lib = ctypes.CDLL(path)
        lib.orc_bf16_to_f32.restype = ctypes.c_float
        lib.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        lib.orc_f16_to_f32.restype = ctypes.c_float
        lib.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.orc_f32_to_bf16.restype = ctypes.c_uint16
        lib.orc_f32_to_bf16.argtypes = [ctypes.c_float]
        lib.orc_f32_to_f16.restype = ctypes.c_uint16
        lib.orc_f32_to_f16.argtypes = [ctypes.c_float]
        lib.orc_convert_f32_to_storage.argtypes = [_f32p, _u16p, _i64, _int]
        lib.orc_convert_storage_to_f32.argtypes = [_u16p, _f32p, _i64, _int]
        lib.orc_rope_table.argtypes = [_f32p, _f32p, _int, _int, _flt, _flt]
        lib.orc_rope.argtypes = [_u16p, _u16p, _u16p, _u16p, _f32p, _f32p, _int, _int, _int,
                                 _int, _int]
        lib.orc_kv_update.argtypes = [_u16p, _u16p, _u16p, _u16p, _u16p, _i32p, _int, _int,
                                      _int, _int, _int, _int, _int]
        lib.orc_slot_offset.restype = _i64
        lib.orc_slot_offset.argtypes = [_i32p, _int, _int, _int, _int, _int, _int, _int]
        lib.orc_flash_decoding.argtypes = [_u16p, _u16p, _u16p, _u16p, _i32p, _int, _int, _int,
                                           _int, _int, _flt, _int, _int, _int]
        lib.orc_decode_batch.argtypes = [_u16p, _i64, _u16p, _i64, _u16p, _u16p, _i32p, _int,
                                         _i32p, _int, _int, _int, _int, _int, _flt, _int, _int,
                                         _int, _int]
        lib.orc_decode_step.argtypes = [_u16p, _i64, _u16p, _i64, _u16p, _u16p, _u16p, _f32p,
                                        _f32p, _u16p, _u16p, _i32p, _int, _i32p, _int, _int,
                                        _int, _int, _int, _flt, _int, _int, _int, _int]
        lib.orc_rmsnorm.argtypes = [_u16p, _u16p, _u16p, _flt, _int, _int]
        lib.orc_silu_mul.argtypes = [_u16p, _int, _int]
        lib.orc_argmax.restype = _int
        lib.orc_argmax.argtypes = [_u16p, _int]
        lib.orc_topk_filter.argtypes = [_u16p, _int, _int, _i32p, _f32p]
        lib.orc_bitonic_desc.argtypes = [_i32p, _f32p, _int]
        lib.orc_top_p_pick.restype = _int
        lib.orc_top_p_pick.argtypes = [_f32p, _int, _flt, _flt, _f32p, _f32p]
        lib.orc_prefill.argtypes = [_u16p, _i64, _u16p, _i64, _u16p, _u16p, _u16p, _f32p, _f32p,
                                    _u16p, _u16p, _i32p, _int, _i32p, _i32p, _int, _int, _int,
                                    _int, _int, _flt, _int, _int, _int, _int]

    # ---- conversions -------------------------------------------------
    def rmsnorm(self, x, weight, eps):
        """RMSNorm of the rows of x (bf16 bits, [rows, cols])."""
        x = np.ascontiguousarray(x)
        out = np.empty_like(x)
        cols = x.shape[-1]
        self.lib.orc_rmsnorm(_ptr(out, "u16"), _ptr(x, "u16"), _ptr(np.ascontiguousarray(weight), "u16"),
                             eps, x.size // cols, cols)
        return out

    def silu_mul(self, gate_up, inter):
        """gate = silu(gate) * up in place on rows [gate | up] (bf16 bits)."""
        assert gate_up.flags["C_CONTIGUOUS"]
        self.lib.orc_silu_mul(_ptr(gate_up, "u16"), gate_up.size // (2 * inter), inter)
        return gate_up

    def argmax(self, x):
        x = np.ascontiguousarray(x)
        return int(self.lib.orc_argmax(_ptr(x, "u16"), x.size))

    # ---- top-k / top-p sampling (sampling_optimized.cu) ---------------
    def topk_filter(self, logits, k_per_block):
        """Candidates of top_k_filter: (keys int32, values f32), 32*k_per_block each."""
        x = np.ascontiguousarray(logits, dtype=np.uint16)
        keys = np.zeros(32 * k_per_block, np.int32)
        vals = np.zeros(32 * k_per_block, np.float32)
        self.lib.orc_topk_filter(_ptr(x, "u16"), x.size, k_per_block, _ptr(keys, "i32"),
                                 _ptr(vals, "f32"))
        return keys, vals

    def bitonic_desc(self, keys, vals):
        """The reference's bitonic network on copies of (keys, vals)."""
        keys = np.array(keys, dtype=np.int32)
        vals = np.array(vals, dtype=np.float32)
        self.lib.orc_bitonic_desc(_ptr(keys, "i32"), _ptr(vals, "f32"), keys.size)
        return keys, vals

    def top_p_pick(self, vals_sorted, top_p, rand_val):
        """(position or -1, prob, cdf) of the sample step on sorted values."""
        v = np.ascontiguousarray(vals_sorted, dtype=np.float32)
        prob = np.empty_like(v)
        cdf = np.empty_like(v)
        i = self.lib.orc_top_p_pick(_ptr(v, "f32"), v.size, top_p, rand_val, _ptr(prob, "f32"),
                                    _ptr(cdf, "f32"))
        return int(i), prob, cdf

    def sort_and_sample(self, logits, top_p, top_k, rand_val):
        """apply_sort_and_sample: dict(keys, vals) of the sorted candidates,
        token (None when no candidate's interval holds the target), prob, cdf."""
        keys, vals = self.topk_filter(logits, top_k // 32)
        keys, vals = self.bitonic_desc(keys, vals)
        i, prob, cdf = self.top_p_pick(vals, top_p, rand_val)
        return dict(keys=keys, vals=vals, token=None if i < 0 else int(keys[i]), pos=i, prob=prob,
                    cdf=cdf)

    def to_storage(self, x: np.ndarray, dtype) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.shape, dtype=np.uint16)
        self.lib.orc_convert_f32_to_storage(_ptr(x, "f32"), _ptr(out, "u16"), x.size, _dt(dtype))
        return out

    def to_f32(self, h: np.ndarray, dtype) -> np.ndarray:
        h = np.ascontiguousarray(h, dtype=np.uint16)
        out = np.empty(h.shape, dtype=np.float32)
        self.lib.orc_convert_storage_to_f32(_ptr(h, "u16"), _ptr(out, "f32"), h.size, _dt(dtype))
        return out

    # ---- path functions ---------------------------------------------
    def rope_table(self, max_pos, head_dim, base=1e6, scale_factor=None):
        cos = np.empty((max_pos, head_dim // 2), np.float32)
        sin = np.empty((max_pos, head_dim // 2), np.float32)
        self.lib.orc_rope_table(_ptr(cos, "f32"), _ptr(sin, "f32"), max_pos, head_dim, base,
                                scale_factor if scale_factor else 0.0)
        return cos, sin

    def rope(self, q, q_bias, k, k_bias, cos, sin, pos, head_dim, hq, hkv, dtype):
        self.lib.orc_rope(_ptr(q, "u16"), _ptr(q_bias, "u16"), _ptr(k, "u16"),
                          _ptr(k_bias, "u16"), _ptr(cos, "f32"), _ptr(sin, "f32"), pos, head_dim,
                          hq, hkv, _dt(dtype))

    def kv_update(self, k_pool, v_pool, k, v, v_bias, table, layer, pos, num_layers, hkv,
                  head_dim, block_size, dtype):
        self.lib.orc_kv_update(_ptr(k_pool, "u16"), _ptr(v_pool, "u16"), _ptr(k, "u16"),
                               _ptr(v, "u16"), _ptr(v_bias, "u16"), _ptr(table, "i32"), layer,
                               pos, num_layers, hkv, head_dim, block_size, _dt(dtype))

    def slot_offset(self, table, pos, layer, kv_head, num_layers, hkv, head_dim, block_size):
        return self.lib.orc_slot_offset(_ptr(table, "i32"), pos, layer, kv_head, num_layers, hkv,
                                        head_dim, block_size)

    def flash_decoding(self, q, k_pool, v_pool, table, layer, hq, hkv, head_dim, pos, sm_scale,
                       block_size, num_layers, dtype):
        out = np.empty((hq, head_dim), np.uint16)
        self.lib.orc_flash_decoding(_ptr(out, "u16"), _ptr(q, "u16"), _ptr(k_pool, "u16"),
                                    _ptr(v_pool, "u16"), _ptr(table, "i32"), layer, hq, hkv,
                                    head_dim, pos, sm_scale, block_size, num_layers, _dt(dtype))
        return out

    def decode_batch(self, q, k_pool, v_pool, tables, positions, layer, hq, hkv, head_dim,
                     sm_scale, block_size, num_layers, dtype, threads=0):
        batch = positions.shape[0]
        q2 = q.reshape(batch, -1)
        out = np.empty((batch, hq * head_dim), np.uint16)
        self.lib.orc_decode_batch(_ptr(out, "u16"), out.shape[1], _ptr(q2, "u16"), q2.shape[1],
                                  _ptr(k_pool, "u16"), _ptr(v_pool, "u16"), _ptr(tables, "i32"),
                                  tables.shape[1], _ptr(positions, "i32"), batch, layer, hq, hkv,
                                  head_dim, sm_scale, block_size, num_layers, _dt(dtype), threads)
        return out.reshape(batch, hq, head_dim)

    def decode_step(self, qkv, q_bias, k_bias, v_bias, cos, sin, k_pool, v_pool, tables,
                    positions, layer, hq, hkv, head_dim, sm_scale, block_size, num_layers, dtype,
                    threads=0):
        """In place on qkv [B, (hq+2hkv)*d] and the pools; returns out [B, hq, d]."""
        batch = positions.shape[0]
        out = np.empty((batch, hq * head_dim), np.uint16)
        self.lib.orc_decode_step(_ptr(out, "u16"), out.shape[1], _ptr(qkv, "u16"), qkv.shape[1],
                                 _ptr(q_bias, "u16"), _ptr(k_bias, "u16"), _ptr(v_bias, "u16"),
                                 _ptr(cos, "f32"), _ptr(sin, "f32"), _ptr(k_pool, "u16"),
                                 _ptr(v_pool, "u16"), _ptr(tables, "i32"), tables.shape[1],
                                 _ptr(positions, "i32"), batch, layer, hq, hkv, head_dim,
                                 sm_scale, block_size, num_layers, _dt(dtype), threads)
        return out.reshape(batch, hq, head_dim)

    def prefill(self, qkv, q_bias, k_bias, v_bias, cos, sin, k_pool, v_pool, tables, cu_seqlens,
                start_pos, layer, hq, hkv, head_dim, sm_scale, block_size, num_layers, dtype,
                threads=0):
        """In place on qkv [T, (hq+2hkv)*d] and the pools; returns out [T, hq, d]."""
        batch = start_pos.shape[0]
        total = int(cu_seqlens[-1])
        out = np.empty((total, hq * head_dim), np.uint16)
        self.lib.orc_prefill(_ptr(out, "u16"), out.shape[1], _ptr(qkv, "u16"), qkv.shape[1],
                             _ptr(q_bias, "u16"), _ptr(k_bias, "u16"), _ptr(v_bias, "u16"),
                             _ptr(cos, "f32"), _ptr(sin, "f32"), _ptr(k_pool, "u16"),
                             _ptr(v_pool, "u16"), _ptr(tables, "i32"), tables.shape[1],
                             _ptr(cu_seqlens, "i32"), _ptr(start_pos, "i32"), batch, layer, hq,
                             hkv, head_dim, sm_scale, block_size, num_layers, _dt(dtype), threads)
        return out.reshape(total, hq, head_dim)


_ORACLE = None


def get() -> Oracle:
    global _ORACLE
    if _ORACLE is None:
        _ORACLE = Oracle()
    return _ORACLE
