"""ctypes binding of liblucattn.so (include/luc_attn.h) over torch tensors.

torch is imported first so that the library binds to the HIP runtime torch has
already loaded (both name it libamdhip64.so.7): device pointers and streams
from torch are then valid in the library.
"""
from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))

LUC_BF16 = 0
LUC_F16 = 1
STATUS = {0: "LUC_OK", -1: "LUC_E_INVALID", -2: "LUC_E_UNSUPPORTED", -3: "LUC_E_LOAD",
          -4: "LUC_E_HIP", -5: "LUC_E_WORKSPACE", -6: "LUC_E_NOMEM"}

_vp = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); every function declared in include/luc_attn.h
SIGNATURES = {
    "luc_abi_version": (_i32, []),
    "luc_last_error": (ctypes.c_char_p, []),
    "luc_init": (_i32, [_i32, ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "luc_destroy": (None, [_vp]),
    "luc_rope_table": (_i32, [_vp, _vp, _i32, _i32, _f32, _f32]),
    "luc_rope": (_i32, [_vp, _vp, _i32, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _i32, _i32, _i32,
                        _i32]),
    "luc_kv_cache_update": (_i32, [_vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _i32, _i32,
                                   _vp, _i32, _i32, _i32, _i32, _i32, _i32]),
    "luc_rope_append": (_i32, [_vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _vp,
                               _vp, _i32, _i32, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32,
                               _i32]),
    "luc_paged_decode_workspace_size": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "luc_paged_decode": (_i32, [_vp, _vp, _i32, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i32, _i32,
                                _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _i32,
                                _vp, _sz]),
    "luc_decode_step": (_i32, [_vp, _vp, _i32, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                               _i32, _i32, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                               _f32, _i32, _vp, _i64, _vp, _sz]),
    "luc_decode_step_noalloc": (_i32, [_vp, _vp, _i32, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp,
                                       _vp, _vp, _i32, _i32, _vp, _i32, _i32, _i32, _i32, _i32,
                                       _i32, _i32, _i32, _f32, _i32, _vp, _i64]),
    "luc_paged_prefill": (_i32, [_vp, _vp, _i32, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                 _vp, _i32, _i32, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32,
                                 _i32, _i32, _i32, _f32, _vp, _i64]),
    "luc_rmsnorm": (_i32, [_vp, _vp, _i32, _vp, _vp, _vp, _f32, _i32, _i32]),
    "luc_silu_mul": (_i32, [_vp, _vp, _i32, _vp, _i32, _i32]),
    "luc_gemv": (_i32, [_vp, _vp, _i32, _vp, _vp, _vp, _vp, _i32, _i32]),
    "luc_rmsnorm_gemv": (_i32, [_vp, _vp, _i32, _vp, _vp, _vp, _f32, _vp, _vp, _i32, _i32]),
    "luc_gate_up_silu": (_i32, [_vp, _vp, _i32, _vp, _vp, _vp, _f32, _vp, _i32, _i32]),
    "luc_embedding": (_i32, [_vp, _vp, _i32, _vp, _vp, _vp, _i32, _i32, _i32]),
    "luc_argmax": (_i32, [_vp, _vp, _i32, _vp, _i32, _vp]),
    "luc_sort_and_sample": (_i32, [_vp, _vp, _i32, _vp, _i32, _f32, _i32, _f32, _vp, _sz, _vp]),
    "luc_gather_floor": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _vp, _i32, _i32, _i32, _i32,
                                _i32, _i32, _vp]),
    "luc_stream_read": (_i32, [_vp, _vp, _vp, _sz, _vp]),
    "luc_blocks_create": (_i32, [_i32, _i32, _i32, ctypes.POINTER(_vp)]),
    "luc_blocks_destroy": (None, [_vp]),
    "luc_blocks_reserve": (_i32, [_vp, _i32, _i32]),
    "luc_blocks_reserve_batch": (_i32, [_vp, _i32, _vp, _vp]),
    "luc_blocks_release": (_i32, [_vp, _i32]),
    "luc_blocks_num_free": (_i32, [_vp]),
    "luc_blocks_num_pages": (_i32, [_vp, _i32]),
    "luc_blocks_table": (_i32, [_vp, _i32, _i32, _vp, _i32]),
}


def lib_dir() -> str:
    """Directory of the gfx950 code objects (and of liblucattn.so)."""
    return os.path.join(_HERE, "lib")


def lib_path() -> str:
    """liblucattn.so in lib/, or LUC_LIB_PATH: another build of the same
    sources (the CPU sanitizer build of sanitize.py)."""
    return os.environ.get("LUC_LIB_PATH") or os.path.join(lib_dir(), "liblucattn.so")


class LucError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"{STATUS.get(code, code)}: {msg}")
        self.code = code


_CDLL = None


def load_cdll() -> ctypes.CDLL:
    """Load liblucattn.so and declare its signatures (no GPU call)."""
    global _CDLL
    if _CDLL is None:
        path = lib_path()
        if not os.path.exists(path):
            raise LucError(-3, f"{path} is not built (run lucciola-rs_amd/build.py)")
        cdll = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(cdll, name)
            fn.restype = res
            fn.argtypes = args
        _CDLL = cdll
    return _CDLL


def dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return LUC_BF16
    if t.dtype == torch.float16:
        return LUC_F16
    raise TypeError(f"unsupported storage dtype {t.dtype}")


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def pool_pages(pool, num_layers, num_kv_heads, head_dim) -> int:
    """Pages in a K/V pool tensor ([pages][layers][kv heads][16][head_dim], or
    the same elements flat)."""
    if pool.dim() == 5:
        return int(pool.shape[0])
    return int(pool.numel() // (num_layers * num_kv_heads * 16 * head_dim))


def _stream(stream):
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


class LucAttn:
    """One luc_ctx (code objects loaded on one device) and its entry points."""

    def __init__(self, device: int = 0):
        self.lib = load_cdll()
        self.device = device
        self.ctx = ctypes.c_void_p()
        with torch.cuda.device(device):
            rc = self.lib.luc_init(device, lib_dir().encode(), ctypes.byref(self.ctx))
        self._check(rc)

    def close(self):
        if self.ctx:
            self.lib.luc_destroy(self.ctx)
            self.ctx = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc):
        if rc != 0:
            raise LucError(rc, self.lib.luc_last_error().decode())

    # ---- host helpers --------------------------------------------------
    def rope_table(self, max_pos, head_dim, base=1e6, scale_factor=None):
        cos = torch.empty((max_pos, head_dim // 2), dtype=torch.float32)
        sin = torch.empty((max_pos, head_dim // 2), dtype=torch.float32)
        self._check(self.lib.luc_rope_table(_p(cos), _p(sin), max_pos, head_dim, base,
                                            scale_factor or 0.0))
        return cos, sin

    def workspace_size(self, batch, hq, hkv, head_dim, max_ctx, split_tokens=0):
        return self.lib.luc_paged_decode_workspace_size(batch, hq, hkv, head_dim, max_ctx,
                                                        split_tokens)

    # ---- launches ------------------------------------------------------
    def rope(self, q, q_bias, k, k_bias, row_stride, cos, sin, positions, num_tokens, hq, hkv,
             head_dim, stream=None):
        self._check(self.lib.luc_rope(self.ctx, _stream(stream), dtype_code(q), _p(q), _p(q_bias),
                                      _p(k), _p(k_bias), row_stride, _p(cos), _p(sin),
                                      _p(positions), num_tokens, hq, hkv, head_dim))

    def kv_cache_update(self, k_pool, v_pool, k, v, v_bias, row_stride, tables, positions,
                        num_tokens, layer, num_layers, hkv, head_dim, block_size=16,
                        stream=None, num_blocks=None):
        nb = num_blocks if num_blocks is not None else pool_pages(k_pool, num_layers, hkv, head_dim)
        self._check(self.lib.luc_kv_cache_update(
            self.ctx, _stream(stream), dtype_code(k_pool), _p(k_pool), _p(v_pool), _p(k), _p(v),
            _p(v_bias), row_stride, _p(tables), tables.shape[-1], nb, _p(positions), num_tokens,
            layer, num_layers, hkv, head_dim, block_size))

    def rope_append(self, q, q_bias, k, k_bias, v, v_bias, row_stride, cos, sin, positions,
                    tables, k_pool, v_pool, num_tokens, layer, num_layers, hq, hkv, head_dim,
                    block_size=16, stream=None, num_blocks=None):
        nb = num_blocks if num_blocks is not None else pool_pages(k_pool, num_layers, hkv, head_dim)
        self._check(self.lib.luc_rope_append(
            self.ctx, _stream(stream), dtype_code(k_pool), _p(q), _p(q_bias), _p(k), _p(k_bias),
            _p(v), _p(v_bias), row_stride, _p(cos), _p(sin), _p(positions), _p(tables),
            tables.shape[-1], nb, _p(k_pool), _p(v_pool), num_tokens, layer, num_layers, hq, hkv,
            head_dim, block_size))

    def paged_decode(self, out, q, k_pool, v_pool, tables, positions, batch, max_ctx, layer,
                     num_layers, hq, hkv, head_dim, sm_scale, split_tokens=0, workspace=None,
                     out_row_stride=None, q_row_stride=None, block_size=16, stream=None,
                     num_blocks=None):
        ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        nb = num_blocks if num_blocks is not None else pool_pages(k_pool, num_layers, hkv, head_dim)
        self._check(self.lib.luc_paged_decode(
            self.ctx, _stream(stream), dtype_code(k_pool), _p(out),
            out_row_stride if out_row_stride is not None else hq * head_dim, _p(q),
            q_row_stride if q_row_stride is not None else hq * head_dim, _p(k_pool), _p(v_pool),
            _p(tables), tables.shape[-1], nb, _p(positions), batch, max_ctx, layer, num_layers, hq,
            hkv, head_dim, block_size, sm_scale, split_tokens, _p(workspace), ws_bytes))


    def decode_step(self, qkv, q_bias, k_bias, v_bias, cos, sin, k_pool, v_pool, tables,
                    positions, batch, max_ctx, layer, num_layers, hq, hkv, head_dim, sm_scale,
                    out, workspace=None, split_tokens=0, qkv_row_stride=None,
                    out_row_stride=None, block_size=16, stream=None, num_blocks=None):
        ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        nb = num_blocks if num_blocks is not None else pool_pages(k_pool, num_layers, hkv, head_dim)
        self._check(self.lib.luc_decode_step(
            self.ctx, _stream(stream), dtype_code(k_pool), _p(qkv),
            qkv_row_stride if qkv_row_stride is not None else (hq + 2 * hkv) * head_dim,
            _p(q_bias), _p(k_bias), _p(v_bias), _p(cos), _p(sin), _p(k_pool), _p(v_pool),
            _p(tables), tables.shape[-1], nb, _p(positions), batch, max_ctx, layer, num_layers, hq, hkv,
            head_dim, block_size, sm_scale, split_tokens, _p(out),
            out_row_stride if out_row_stride is not None else hq * head_dim, _p(workspace),
            ws_bytes))

    def decode_step_noalloc(self, qkv, q_bias, k_bias, v_bias, cos, sin, k_pool, v_pool, tables,
                            positions, batch, max_ctx, layer, num_layers, hq, hkv, head_dim,
                            sm_scale, out, split_tokens=0, qkv_row_stride=None,
                            out_row_stride=None, block_size=16, stream=None, num_blocks=None):
        """luc_decode_step_noalloc: luc_decode_step with the library's fixed
        per-device scratch as its split-K workspace (no workspace argument)."""
        nb = num_blocks if num_blocks is not None else pool_pages(k_pool, num_layers, hkv, head_dim)
        self._check(self.lib.luc_decode_step_noalloc(
            self.ctx, _stream(stream), dtype_code(k_pool), _p(qkv),
            qkv_row_stride if qkv_row_stride is not None else (hq + 2 * hkv) * head_dim,
            _p(q_bias), _p(k_bias), _p(v_bias), _p(cos), _p(sin), _p(k_pool), _p(v_pool),
            _p(tables), tables.shape[-1], nb, _p(positions), batch, max_ctx, layer, num_layers, hq, hkv,
            head_dim, block_size, sm_scale, split_tokens, _p(out),
            out_row_stride if out_row_stride is not None else hq * head_dim))

    def paged_prefill(self, qkv, q_bias, k_bias, v_bias, cos, sin, k_pool, v_pool, tables,
                      cu_seqlens, start_pos, total_rows, max_ctx, layer, num_layers, hq, hkv,
                      head_dim, sm_scale, out, qkv_row_stride=None, out_row_stride=None,
                      block_size=16, stream=None, num_blocks=None):
        """luc_paged_prefill: rope + cache write + causal attention of packed
        prompts (cu_seqlens [B+1], start_pos [B] device int32)."""
        nb = num_blocks if num_blocks is not None else pool_pages(k_pool, num_layers, hkv, head_dim)
        self._check(self.lib.luc_paged_prefill(
            self.ctx, _stream(stream), dtype_code(k_pool), _p(qkv),
            qkv_row_stride if qkv_row_stride is not None else (hq + 2 * hkv) * head_dim,
            _p(q_bias), _p(k_bias), _p(v_bias), _p(cos), _p(sin), _p(k_pool), _p(v_pool),
            _p(tables), tables.shape[-1], nb, _p(cu_seqlens), _p(start_pos), start_pos.shape[0],
            total_rows, max_ctx, layer, num_layers, hq, hkv, head_dim, block_size, sm_scale,
            _p(out), out_row_stride if out_row_stride is not None else hq * head_dim))

    # ---- the model loop's small kernels ----
    def rmsnorm(self, out, x, weight, eps, stream=None):
        """luc_rmsnorm over the rows of x ([rows, cols] bf16); out may be x."""
        cols = x.shape[-1]
        self._check(self.lib.luc_rmsnorm(self.ctx, _stream(stream), dtype_code(x), _p(out), _p(x),
                                         _p(weight), eps, x.numel() // cols, cols))

    @staticmethod
    def _gemv_shapes(name, y, x, w, residual):
        n, k = w.shape
        if not (w.is_contiguous() and x.is_contiguous() and y.is_contiguous()) or \
                x.numel() != k or y.numel() != n or \
                (residual is not None and (residual.numel() != n or not residual.is_contiguous())):
            raise ValueError(f"{name}: w {tuple(w.shape)}, x {tuple(x.shape)}, y {tuple(y.shape)}: "
                             "want contiguous x [k], y [n] (and residual [n]) for w [n, k]")
        return n, k

    def gemv(self, y, x, w, residual=None, stream=None):
        """luc_gemv: y = x w^T (+ residual) for one row x [k] (or [1, k]) and
        w [n, k] bf16; residual may be y (an in-place residual add)."""
        n, k = self._gemv_shapes("gemv", y, x, w, residual)
        self._check(self.lib.luc_gemv(self.ctx, _stream(stream), dtype_code(w), _p(y), _p(x), _p(w),
                                      _p(residual), n, k))

    def rmsnorm_gemv(self, y, x, norm_weight, eps, w, residual=None, stream=None):
        """luc_rmsnorm_gemv: y = rmsnorm(x) w^T (+ residual), one row x [k]."""
        n, k = self._gemv_shapes("rmsnorm_gemv", y, x, w, residual)
        if norm_weight.numel() != k:
            raise ValueError(f"rmsnorm_gemv: norm weight of {norm_weight.numel()}, k {k}")
        self._check(self.lib.luc_rmsnorm_gemv(self.ctx, _stream(stream), dtype_code(w), _p(y), _p(x),
                                              _p(norm_weight), eps, _p(w), _p(residual), n, k))

    def gate_up_silu(self, act, x, norm_weight, eps, w, stream=None):
        """luc_gate_up_silu: act [I] = silu(g) * u of [g | u] = rmsnorm(x) w^T
        (x itself when norm_weight is None), w [2 I, k] = [gate; up]."""
        two_i, k = w.shape
        if two_i % 2 or not (w.is_contiguous() and x.is_contiguous() and act.is_contiguous()) or \
                x.numel() != k or act.numel() != two_i // 2 or \
                (norm_weight is not None and norm_weight.numel() != k):
            raise ValueError(f"gate_up_silu: w {tuple(w.shape)}, x {tuple(x.shape)}, act {tuple(act.shape)}: "
                             "want contiguous x [k], act [I] for w [2 I, k]")
        self._check(self.lib.luc_gate_up_silu(self.ctx, _stream(stream), dtype_code(w), _p(act), _p(x),
                                              _p(norm_weight), eps, _p(w), two_i // 2, k))

    def silu_mul(self, gate_up, intermediate, stream=None):
        """luc_silu_mul in place on [rows, 2*intermediate] (gate | up) rows."""
        rows = gate_up.numel() // (2 * intermediate)
        self._check(self.lib.luc_silu_mul(self.ctx, _stream(stream), dtype_code(gate_up),
                                          _p(gate_up), rows, intermediate))

    def embedding(self, out, table, ids, stream=None):
        """luc_embedding: out[t] = table[ids[t]] (ids: device int32/uint32)."""
        self._check(self.lib.luc_embedding(self.ctx, _stream(stream), dtype_code(table), _p(out),
                                           _p(table), _p(ids), ids.numel(), table.shape[0],
                                           table.shape[1]))

    def gather_floor(self, k_pool, v_pool, tables, positions, batch, max_ctx, layer, num_layers,
                     hkv, head_dim, sink, stream=None):
        """luc_gather_floor: the decode step's K/V page slabs read with its work
        split and no arithmetic (sink: a one-element device int32 tensor)."""
        self._check(self.lib.luc_gather_floor(
            self.ctx, _stream(stream), _p(k_pool), _p(v_pool), _p(tables), tables.shape[-1],
            pool_pages(k_pool, num_layers, hkv, head_dim), _p(positions), batch, max_ctx, layer,
            num_layers, hkv, head_dim, _p(sink)))

    def stream_read(self, src, sink, stream=None):
        """luc_stream_read of the whole of src (a contiguous device tensor)."""
        self._check(self.lib.luc_stream_read(self.ctx, _stream(stream), _p(src),
                                             src.numel() * src.element_size(), _p(sink)))

    def argmax(self, logits, out_idx, stream=None):
        """luc_argmax into out_idx (a one-element device int32 tensor)."""
        self._check(self.lib.luc_argmax(self.ctx, _stream(stream), dtype_code(logits), _p(logits),
                                        logits.numel(), _p(out_idx)))

    def sort_and_sample(self, logits, top_p, top_k, rand_val, sort_buffer, out_idx, stream=None):
        """luc_sort_and_sample of one bf16 logits row into out_idx (one-element
        device int32 tensor, left unwritten when no candidate is drawn);
        sort_buffer (>= 8*top_k bytes of device memory) returns the sorted
        (index, value) candidates."""
        self._check(self.lib.luc_sort_and_sample(
            self.ctx, _stream(stream), dtype_code(logits), _p(logits), logits.numel(), float(top_p),
            int(top_k), float(rand_val), _p(sort_buffer),
            sort_buffer.numel() * sort_buffer.element_size(), _p(out_idx)))

    def workspace(self, batch, hq, hkv, head_dim, max_ctx, split_tokens=0, device=None):
        """A zero-filled decode workspace (None when no split-K is needed)."""
        need = self.workspace_size(batch, hq, hkv, head_dim, max_ctx, split_tokens)
        if need == 0:
            return None
        return torch.zeros(need // 4, dtype=torch.float32,
                           device=device if device is not None else f"cuda:{self.device}")


_DEFAULT = {}


def default(device: int = 0) -> LucAttn:
    """Process-wide LucAttn for `device` (created on first use)."""
    if device not in _DEFAULT:
        _DEFAULT[device] = LucAttn(device)
    return _DEFAULT[device]
