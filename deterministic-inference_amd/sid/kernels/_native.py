"""ctypes binding of libsid_hip.so: torch tensors in, raw device pointers out.

Each method checks its tensors the way the reference's TORCH_CHECKs do
(sid/csrc/flash_decode.cu:325-345, 386-395) and raises RuntimeError on a violation or on
a non-zero status from the library (message from `sid_last_error()`). Launches go on
torch's current stream of the tensors' device, so they order with surrounding torch work
and are captured by `torch.cuda.graph` like any torch op.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

_i32, _i64, _f32, _vp = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p

# name -> argtypes (every entry point returns int status)
_SIGNATURES = {
    "sid_reshape_and_cache": [_vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i64, _vp],
    "sid_flash_decode_fwd": [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i64, _i32,
                             _i32, _f32, _vp, _vp, _i32, _i32, _vp, _vp],
    "sid_extend_attention_fwd": [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i32, _i32, _i32,
                                 _i64, _i32, _i32, _f32, _vp, _i64, _vp, _vp],
    "sid_rmsnorm": [_vp, _vp, _vp, _i64, _i32, _f32, _vp],
    "sid_fused_add_rmsnorm": [_vp, _vp, _vp, _i64, _i32, _f32, _vp],
    "sid_rope_apply": [_vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i64, _vp],
    "sid_linear": [_vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _vp],
    "sid_linear_partials": [_vp, _i64, _vp, _vp, _i64, _i64, _i64, _vp],
    "sid_fused_add_rmsnorm_partials": [_vp, _i32, _vp, _vp, _vp, _i64, _i32, _f32, _vp],
    "sid_silu_mul_partials": [_vp, _i32, _vp, _i64, _i64, _vp],
    "sid_qkv_post": [_vp, _vp, _i32, _i64, _i32, _i32, _i32, _vp, _vp, _f32, _vp, _vp, _i64, _vp,
                     _vp, _vp, _vp, _i64, _vp],
    "sid_silu_mul": [_vp, _vp, _i64, _i64, _vp],
    "sid_linear_silu_mul": [_vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "sid_gather_rows": [_vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "sid_argmax_rows": [_vp, _i64, _vp, _i64, _i64, _vp],
    "sid_build_paged_decode_indices": [_vp, _i64, _i64, _i32, _vp, _vp, _vp, _vp, _i32, _vp],
    "sid_flash_decode_segments_fwd": [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i64,
                                      _i32, _i32, _i32, _i32, _i32, _vp, _f32, _vp, _vp, _i32,
                                      _i32, _vp, _vp],
    "sid_flash_decode_workers_fwd": [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i64,
                                     _i32, _i32, _i32, _i32, _i32, _vp, _f32, _vp, _vp, _i32,
                                     _i32, _vp, _i32, _vp],
    "sid_flash_decode_segments_fwd_noalloc": [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32,
                                              _i32, _i64, _i32, _i32, _i32, _i32, _i32, _vp,
                                              _f32, _vp, _vp],
    "sid_sample_rows": [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _i64, _vp, _vp],
    "sid_linear_sample": [_vp, _i64, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _i64, _vp, _vp,
                          _i32, _vp],
    "sid_linear_argmax": [_vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp],
    "sid_linear_residual": [_vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "sid_rmsnorm_linear_silu_mul": [_vp, _i32, _vp, _f32, _vp, _vp, _i64, _i64, _i64, _vp],
    "sid_rmsnorm_qkv_post": [_vp, _i32, _vp, _f32, _vp, _i64, _i64, _i32, _i32, _i32, _vp, _vp,
                             _vp, _vp, _i64, _vp, _vp, _vp, _vp, _i64, _vp],
    "sid_rmsnorm_f32": [_vp, _vp, _vp, _i64, _i32, _f32, _vp],
    "sid_pack_decode_weight": [_vp, _vp, _i64, _i64, _i32, _vp],
}
EXPORTED = ("sid_last_error", "sid_abi_version", "sid_extend_attention_workspace_bytes",
            "sid_linear_argmax_workspace_bytes", "sid_sample_workspace_bytes",
            "sid_qwen3_extend_workspace_bytes", "sid_qwen3_extend_forward",
            "sid_flash_decode_noalloc_scratch_bytes", "sid_linear_sample_workspace_bytes",
            *_SIGNATURES)
ABI_VERSION = 22


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _gpu(t: torch.Tensor, name: str, dtype: torch.dtype | None = None) -> None:
    _check(isinstance(t, torch.Tensor) and t.is_cuda, f"{name} must be a GPU tensor")
    _check(t.is_contiguous(), f"{name} must be contiguous")
    if dtype is not None:
        _check(t.dtype == dtype, f"{name} must be {dtype}, got {t.dtype}")


def _ptr(t) -> int:
    """Device address of an optional tensor (0 for None)."""
    return 0 if t is None else t.data_ptr()


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


class NativeLib:
    """The loaded library; method names and argument orders follow the reference ops."""

    def __init__(self, path: Path):
        self.path = Path(path)
        self.lib = ctypes.CDLL(str(self.path))
        self.lib.sid_last_error.restype = ctypes.c_char_p
        self.lib.sid_last_error.argtypes = []
        self.lib.sid_abi_version.restype = ctypes.c_int
        self.lib.sid_abi_version.argtypes = []
        self.lib.sid_extend_attention_workspace_bytes.restype = ctypes.c_int64
        self.lib.sid_extend_attention_workspace_bytes.argtypes = [_i32, _i64, _i32, _i32, _i32, _i32]
        self.lib.sid_linear_argmax_workspace_bytes.restype = ctypes.c_int64
        self.lib.sid_linear_argmax_workspace_bytes.argtypes = [_i64]
        self.lib.sid_sample_workspace_bytes.restype = ctypes.c_int64
        self.lib.sid_sample_workspace_bytes.argtypes = [_i64, _i64]
        self.lib.sid_linear_sample_workspace_bytes.restype = ctypes.c_int64
        self.lib.sid_linear_sample_workspace_bytes.argtypes = [_i64]
        self.lib.sid_flash_decode_noalloc_scratch_bytes.restype = ctypes.c_int64
        self.lib.sid_flash_decode_noalloc_scratch_bytes.argtypes = []
        for name, argtypes in _SIGNATURES.items():
            fn = getattr(self.lib, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int
        ver = self.lib.sid_abi_version()
        _check(ver == ABI_VERSION, f"libsid_hip.so ABI {ver} != expected {ABI_VERSION}; rebuild")

    def _call(self, name: str, *args) -> None:
        rc = getattr(self.lib, name)(*args)
        if rc != 0:
            raise RuntimeError(f"{name}: {self.lib.sid_last_error().decode(errors='replace')}")

    # ---- reference module `sid_flash_decode` (sid/csrc/flash_decode.cu:408-413) ----------

    def flash_decode_fwd(self, q, k_cache, v_cache, kv_indptr, kv_indices, num_splits,
                         max_splits: int, fixed_split_size: int, sm_scale: float,
                         part_o, part_lse, o, segment_size: int = 0,
                         grid_slots: int | None = None, variant: int = 0,
                         wg_order=None, workers: int = 0) -> None:
        """segment_size / grid_slots / variant / wg_order: see sid_flash_decode_segments_fwd
        (defaults: one segment per split, grid of max_splits slots = the reference's
        partition, the default workgroup shape, the grid's own order); workers > 0: stage 1
        by that many workgroups over the items of wg_order (sid_flash_decode_workers_fwd; entries
        flagged ORDER_EMPTY hold no tokens)."""
        _gpu(q, "q", torch.bfloat16)
        _check(q.dim() == 3, "q must be [B, HQ, D]")
        b, hq, d = q.shape
        for name, t in (("k_cache", k_cache), ("v_cache", v_cache)):
            _gpu(t, name, torch.bfloat16)
            _check(t.dim() == 3 and t.shape[2] == d, f"{name} must be [slots, HKV, {d}]")
        _check(k_cache.shape == v_cache.shape, "k_cache and v_cache shapes differ")
        hkv = k_cache.shape[1]
        _gpu(kv_indptr, "kv_indptr", torch.int32)
        _check(kv_indptr.numel() == b + 1, "kv_indptr must have B+1 entries")
        _gpu(kv_indices, "kv_indices", torch.int32)
        if num_splits is not None:  # None: derived on the device from the lengths
            _gpu(num_splits, "num_splits", torch.int32)
            _check(num_splits.numel() == b, "num_splits must have B entries")
        _gpu(part_o, "part_o", torch.float32)
        _gpu(part_lse, "part_lse", torch.float32)
        _check(part_o.dim() == 4 and part_o.shape[1] == hq and part_o.shape[3] == d,
               "part_o workspace too small / wrong shape")
        _check(part_lse.dim() == 3 and part_lse.shape[1] == hq
               and part_lse.shape[2] == part_o.shape[2] and part_lse.shape[0] >= part_o.shape[0],
               "part_lse workspace shape mismatch")
        _gpu(o, "o", torch.bfloat16)
        _check(o.shape == q.shape, "o must have q's shape")
        slots = int(max_splits) if grid_slots is None else int(grid_slots)
        order = self._order_ptr(wg_order, b * slots)
        _check(workers == 0 or wg_order is not None, "a worker launch needs wg_order")
        self._call("sid_flash_decode_workers_fwd", q.data_ptr(), k_cache.data_ptr(),
                   v_cache.data_ptr(), kv_indptr.data_ptr(), kv_indices.data_ptr(),
                   _ptr(num_splits), b, hq, hkv, d, k_cache.shape[0], int(max_splits),
                   int(fixed_split_size), int(segment_size), slots, int(variant), order,
                   float(sm_scale),
                   part_o.data_ptr(), part_lse.data_ptr(), part_o.shape[0], part_o.shape[2],
                   o.data_ptr(), int(workers), _stream(q))

    def flash_decode_fwd_noalloc(self, q, k_cache, v_cache, kv_indptr, kv_indices, num_splits,
                                 max_splits: int, fixed_split_size: int, sm_scale: float, o,
                                 segment_size: int = 0, grid_slots: int | None = None,
                                 variant: int = 0, wg_order=None) -> None:
        """flash_decode_fwd with the split partials in the library's static per-GPU scratch
        (no workspace argument, nothing allocated). Calls that overlap on one GPU race."""
        _gpu(q, "q", torch.bfloat16)
        _check(q.dim() == 3, "q must be [B, HQ, D]")
        b, hq, d = q.shape
        for name, t in (("k_cache", k_cache), ("v_cache", v_cache)):
            _gpu(t, name, torch.bfloat16)
            _check(t.dim() == 3 and t.shape[2] == d, f"{name} must be [slots, HKV, {d}]")
        _check(k_cache.shape == v_cache.shape, "k_cache and v_cache shapes differ")
        _gpu(kv_indptr, "kv_indptr", torch.int32)
        _check(kv_indptr.numel() == b + 1, "kv_indptr must have B+1 entries")
        _gpu(kv_indices, "kv_indices", torch.int32)
        if num_splits is not None:  # None: derived on the device from the lengths
            _gpu(num_splits, "num_splits", torch.int32)
            _check(num_splits.numel() == b, "num_splits must have B entries")
        _gpu(o, "o", torch.bfloat16)
        _check(o.shape == q.shape, "o must have q's shape")
        slots = int(max_splits) if grid_slots is None else int(grid_slots)
        order = self._order_ptr(wg_order, b * slots)
        self._call("sid_flash_decode_segments_fwd_noalloc", q.data_ptr(), k_cache.data_ptr(),
                   v_cache.data_ptr(), kv_indptr.data_ptr(), kv_indices.data_ptr(),
                   _ptr(num_splits), b, hq, k_cache.shape[1], d, k_cache.shape[0],
                   int(max_splits), int(fixed_split_size), int(segment_size), slots,
                   int(variant), order, float(sm_scale), o.data_ptr(), _stream(q))

    @staticmethod
    def _order_ptr(wg_order, n: int) -> int:
        if wg_order is None:
            return 0
        _gpu(wg_order, "wg_order", torch.int32)
        _check(wg_order.numel() >= n, "wg_order must have B * grid_slots entries")
        return wg_order.data_ptr()

    def reshape_and_cache(self, k, v, k_cache, v_cache, slot_mapping) -> None:
        _gpu(k, "k", torch.bfloat16)
        _gpu(v, "v", torch.bfloat16)
        _check(v.shape == k.shape, "v must have k's shape")
        _gpu(k_cache, "k_cache", torch.bfloat16)
        _gpu(v_cache, "v_cache", torch.bfloat16)
        _check(k_cache.shape == v_cache.shape and k_cache.dim() == 3, "bad cache shapes")
        _check(k.dim() == 3 and k.shape[1:] == k_cache.shape[1:],
               "k must be [T, HKV, D] matching the cache")
        _gpu(slot_mapping, "slot_mapping", torch.int64)
        _check(slot_mapping.numel() == k.shape[0], "slot_mapping must have T entries")
        if k.shape[0] == 0:
            return
        self._call("sid_reshape_and_cache", k.data_ptr(), v.data_ptr(), k_cache.data_ptr(),
                   v_cache.data_ptr(), slot_mapping.data_ptr(), k.shape[0], k_cache.shape[1],
                   k_cache.shape[2], k_cache.shape[0], _stream(k))

    # ---- the rest of the decode path ----------------------------------------------------

    def extend_attention_workspace_bytes(self, batch, total_q, hq, hkv, max_extend_len,
                                         max_kv_len) -> int:
        return int(self.lib.sid_extend_attention_workspace_bytes(
            batch, total_q, hq, hkv, max_extend_len, max_kv_len))

    def extend_attention_fwd(self, q, k_buffer, v_buffer, qo_indptr, kv_indptr, kv_indices,
                             max_extend_len: int, sm_scale: float, o, max_kv_len: int,
                             workspace=None) -> None:
        _gpu(q, "q_extend", torch.bfloat16)
        _check(q.dim() == 3, "q_extend must be [Text, HQ, D]")
        _gpu(k_buffer, "k_buffer", torch.bfloat16)
        _gpu(v_buffer, "v_buffer", torch.bfloat16)
        _check(k_buffer.shape == v_buffer.shape and k_buffer.dim() == 3
               and k_buffer.shape[2] == q.shape[2], "bad KV buffer shapes")
        _gpu(qo_indptr, "qo_indptr", torch.int32)
        _gpu(kv_indptr, "kv_indptr", torch.int32)
        _gpu(kv_indices, "kv_indices", torch.int32)
        _check(qo_indptr.numel() == kv_indptr.numel(), "qo_indptr/kv_indptr length mismatch")
        _gpu(o, "o", torch.bfloat16)
        _check(o.shape == q.shape, "o must have q's shape")
        ws_ptr, ws_bytes = None, 0
        if workspace is not None:
            _gpu(workspace, "workspace", torch.uint8)
            ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel()
        self._call("sid_extend_attention_fwd", q.data_ptr(), k_buffer.data_ptr(),
                   v_buffer.data_ptr(), qo_indptr.data_ptr(), kv_indptr.data_ptr(),
                   kv_indices.data_ptr(), qo_indptr.numel() - 1, q.shape[0], q.shape[1],
                   k_buffer.shape[1], q.shape[2], k_buffer.shape[0], int(max_extend_len),
                   int(max_kv_len), float(sm_scale), ws_ptr, ws_bytes, o.data_ptr(), _stream(q))

    def rmsnorm(self, x, w, out, eps: float) -> None:
        _gpu(x, "x", torch.bfloat16)
        _gpu(w, "weight", torch.bfloat16)
        _gpu(out, "out", torch.bfloat16)
        hidden = x.shape[-1]
        _check(w.numel() == hidden and out.shape == x.shape, "rmsnorm shape mismatch")
        self._call("sid_rmsnorm", x.data_ptr(), w.data_ptr(), out.data_ptr(),
                   x.numel() // max(hidden, 1), hidden, float(eps), _stream(x))

    def fused_add_rmsnorm(self, x, residual, w, eps: float) -> None:
        _gpu(x, "x", torch.bfloat16)
        _gpu(residual, "residual", torch.bfloat16)
        _gpu(w, "weight", torch.bfloat16)
        hidden = x.shape[-1]
        _check(residual.shape == x.shape and w.numel() == hidden, "fused_add_rmsnorm shape mismatch")
        self._call("sid_fused_add_rmsnorm", x.data_ptr(), residual.data_ptr(), w.data_ptr(),
                   x.numel() // max(hidden, 1), hidden, float(eps), _stream(x))

    def rope_apply(self, q, k, positions, cos_sin) -> None:
        _gpu(q, "q", torch.bfloat16)
        _gpu(k, "k", torch.bfloat16)
        _gpu(positions, "positions", torch.int64)
        _gpu(cos_sin, "cos_sin", torch.float32)
        t, hq, d = q.shape
        _check(k.dim() == 3 and k.shape[0] == t and k.shape[2] == d, "k must be [T, HKV, D]")
        _check(positions.numel() == t, "positions must have T entries")
        _check(cos_sin.dim() == 2 and cos_sin.shape[1] == d, "cos_sin must be [max_pos, D]")
        self._call("sid_rope_apply", q.data_ptr(), k.data_ptr(), positions.data_ptr(),
                   cos_sin.data_ptr(), t, hq, k.shape[1], d, cos_sin.shape[0], _stream(q))

    def linear(self, x, w, bias, y, out_fp32: bool) -> None:
        m, k, n = self._linear_check(x, w)
        if bias is not None:
            _gpu(bias, "bias", torch.bfloat16)
            _check(bias.numel() == n, "bias must have N entries")
        _gpu(y, "out", torch.float32 if out_fp32 else torch.bfloat16)
        _check(tuple(y.shape) == (m, n), "out must be [M, N]")
        self._call("sid_linear", x.data_ptr(), x.stride(0) if m > 1 else k, w.data_ptr(),
                   bias.data_ptr() if bias is not None else None, y.data_ptr(), m, n, k,
                   1 if out_fp32 else 0, _stream(x))

    def linear_partials(self, x, w, partials) -> None:
        m, k, n = self._linear_check(x, w)
        _gpu(partials, "partials", torch.float32)
        _check(tuple(partials.shape) == (k // 256, m, n), "partials must be [K/256, M, N]")
        self._call("sid_linear_partials", x.data_ptr(), x.stride(0) if m > 1 else k,
                   w.data_ptr(), partials.data_ptr(), m, n, k, _stream(x))

    def linear_argmax_workspace_bytes(self, m: int) -> int:
        return int(self.lib.sid_linear_argmax_workspace_bytes(m))

    def linear_argmax(self, x, w, bias, logits, workspace, out) -> None:
        m, k, n = self._linear_check(x, w)
        if bias is not None:
            _gpu(bias, "bias", torch.bfloat16)
            _check(bias.numel() == n, "bias must have N entries")
        if logits is not None:
            _gpu(logits, "logits", torch.float32)
            _check(tuple(logits.shape) == (m, n), "logits must be [M, N]")
        _gpu(workspace, "workspace")
        _gpu(out, "out", torch.int64)
        _check(out.numel() == m, "out must have M entries")
        self._call("sid_linear_argmax", x.data_ptr(), x.stride(0) if m > 1 else k, w.data_ptr(),
                   bias.data_ptr() if bias is not None else None,
                   logits.data_ptr() if logits is not None else None, m, n, k,
                   workspace.data_ptr(), workspace.numel() * workspace.element_size(),
                   out.data_ptr(), _stream(x))

    def linear_sample_workspace_bytes(self, m: int) -> int:
        return int(self.lib.sid_linear_sample_workspace_bytes(m))

    def linear_sample(self, x, w, temperatures, seeds, positions, workspace, out,
                      recompute_all: bool = False, tiles=None, logits=None) -> None:
        """tiles: None = grouping by row count; True = 128-column tiles; False = streaming
        waves."""
        m, k, n = self._linear_check(x, w)
        if logits is not None:
            _gpu(logits, "logits", torch.float32)
            _check(tuple(logits.shape) == (m, n), "logits must be [M, N]")
        for name, t, dt in (("temperatures", temperatures, torch.float32),
                            ("seeds", seeds, torch.int64), ("positions", positions, torch.int64),
                            ("out", out, torch.int64)):
            _gpu(t, name, dt)
            _check(t.numel() == m, f"{name} must have M entries")
        _gpu(workspace, "workspace")
        self._call("sid_linear_sample", x.data_ptr(), x.stride(0) if m > 1 else k, w.data_ptr(),
                   m, n, k, temperatures.data_ptr(), seeds.data_ptr(), positions.data_ptr(),
                   workspace.data_ptr(), workspace.numel() * workspace.element_size(),
                   out.data_ptr(), logits.data_ptr() if logits is not None else None,
                   int(recompute_all) | {None: 0, True: 2, False: 4}[tiles], _stream(x))

    @staticmethod
    def _linear_check(x, w):
        _check(x.is_cuda and x.dtype == torch.bfloat16 and x.dim() == 2 and x.stride(1) == 1,
               "x must be a 2-D bf16 GPU tensor with unit column stride")
        _gpu(w, "weight", torch.bfloat16)
        m, k = x.shape
        _check(w.dim() == 2 and w.shape[1] == k, f"weight must be [N, {k}]")
        return m, k, w.shape[0]

    def fused_add_rmsnorm_partials(self, partials, residual, w, out, eps: float) -> None:
        _gpu(partials, "partials", torch.float32)
        _gpu(residual, "residual", torch.bfloat16)
        _gpu(out, "out", torch.bfloat16)
        _gpu(w, "weight", torch.bfloat16)
        nch, rows, hidden = partials.shape
        _check(tuple(residual.shape) == (rows, hidden) and out.shape == residual.shape
               and w.numel() == hidden, "fused_add_rmsnorm_partials shape mismatch")
        self._call("sid_fused_add_rmsnorm_partials", partials.data_ptr(), nch, residual.data_ptr(),
                   w.data_ptr(), out.data_ptr(), rows, hidden, float(eps), _stream(out))

    def silu_mul_partials(self, partials, out) -> None:
        _gpu(partials, "partials", torch.float32)
        _gpu(out, "out", torch.bfloat16)
        nch, t, two_i = partials.shape
        _check(two_i % 2 == 0 and tuple(out.shape) == (t, two_i // 2), "silu_mul_partials shape")
        self._call("sid_silu_mul_partials", partials.data_ptr(), nch, out.data_ptr(), t,
                   two_i // 2, _stream(out))

    def qkv_post(self, qkv, partials, q_norm, k_norm, eps: float, positions, cos_sin, slots,
                 q_out, k_cache, v_cache) -> None:
        _check((qkv is None) != (partials is None), "give exactly one of qkv and partials")
        if qkv is not None:
            _gpu(qkv, "qkv", torch.bfloat16)
            t, width, nch = qkv.shape[0], qkv.shape[1], 0
        else:
            _gpu(partials, "partials", torch.float32)
            nch, t, width = partials.shape
        _gpu(q_out, "q_out", torch.bfloat16)
        _check(q_out.dim() == 3 and q_out.shape[0] == t, "q_out must be [T, HQ, D]")
        hq, d = q_out.shape[1], q_out.shape[2]
        for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
            _gpu(c, name, torch.bfloat16)
            _check(c.dim() == 3 and c.shape[2] == d, f"{name} must be [S, HKV, D]")
        hkv = k_cache.shape[1]
        _check(width == (hq + 2 * hkv) * d, "projection width != (HQ + 2*HKV) * D")
        _gpu(q_norm, "q_norm", torch.bfloat16)
        _gpu(k_norm, "k_norm", torch.bfloat16)
        _gpu(positions, "positions", torch.int64)
        _gpu(slots, "slots", torch.int64)
        _gpu(cos_sin, "cos_sin", torch.float32)
        _check(positions.numel() == t and slots.numel() == t, "positions/slots must have T entries")
        self._call("sid_qkv_post", qkv.data_ptr() if qkv is not None else None,
                   partials.data_ptr() if partials is not None else None, nch, t, hq, hkv, d,
                   q_norm.data_ptr(), k_norm.data_ptr(), float(eps), positions.data_ptr(),
                   cos_sin.data_ptr(), cos_sin.shape[0], slots.data_ptr(), q_out.data_ptr(),
                   k_cache.data_ptr(), v_cache.data_ptr(), k_cache.shape[0], _stream(q_out))

    def linear_residual(self, x, w, residual, r32) -> None:
        """residual, r32 <- r = residual + bf16(x @ w^T) (fp32 r; residual = bf16(r))."""
        m, k, n = self._linear_check(x, w)
        _gpu(residual, "residual", torch.bfloat16)
        _gpu(r32, "r32", torch.float32)
        _check(tuple(residual.shape) == (m, n) and tuple(r32.shape) == (m, n),
               "residual / r32 must be [M, N]")
        self._call("sid_linear_residual", x.data_ptr(), x.stride(0), w.data_ptr(),
                   residual.data_ptr(), r32.data_ptr(), m, n, k, _stream(r32))

    @staticmethod
    def _norm_src(src):
        _check(src.is_cuda and src.dim() == 2 and src.is_contiguous()
               and src.dtype in (torch.float32, torch.bfloat16),
               "norm source must be a contiguous fp32 or bf16 [M, hidden] GPU tensor")
        return int(src.dtype == torch.float32)

    def rmsnorm_linear_silu_mul(self, src, norm_w, eps: float, w, out) -> None:
        """out <- silu_mul(bf16(rmsnorm(src) * norm_w) @ w^T), w = [gate rows | up rows]."""
        f32 = self._norm_src(src)
        _gpu(norm_w, "norm weight", torch.bfloat16)
        _gpu(w, "weight", torch.bfloat16)
        _gpu(out, "out", torch.bfloat16)
        m, hidden = src.shape
        _check(w.dim() == 2 and w.shape[1] == hidden and w.shape[0] % 2 == 0
               and norm_w.numel() == hidden, "rmsnorm_linear_silu_mul shapes")
        inter = w.shape[0] // 2
        _check(tuple(out.shape) == (m, inter), "out must be [M, I]")
        self._call("sid_rmsnorm_linear_silu_mul", src.data_ptr(), f32, norm_w.data_ptr(),
                   float(eps), w.data_ptr(), out.data_ptr(), m, hidden, inter, _stream(out))

    def rmsnorm_qkv_post(self, src, norm_w, eps: float, w, q_norm, k_norm, positions, cos_sin,
                         slots, q_out, k_cache, v_cache) -> None:
        """qkv_post over bf16(rmsnorm(src) * norm_w) @ w^T (one launch)."""
        f32 = self._norm_src(src)
        m, hidden = src.shape
        _gpu(norm_w, "norm weight", torch.bfloat16)
        _gpu(w, "weight", torch.bfloat16)
        _gpu(q_out, "q_out", torch.bfloat16)
        _check(q_out.dim() == 3 and q_out.shape[0] == m, "q_out must be [M, HQ, D]")
        hq, d = q_out.shape[1], q_out.shape[2]
        for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
            _gpu(c, name, torch.bfloat16)
            _check(c.dim() == 3 and c.shape[2] == d, f"{name} must be [S, HKV, D]")
        hkv = k_cache.shape[1]
        _check(w.dim() == 2 and w.shape[0] == (hq + 2 * hkv) * d and w.shape[1] == hidden
               and norm_w.numel() == hidden, "qkv weight must be [(HQ + 2*HKV) * D, hidden]")
        _gpu(q_norm, "q_norm", torch.bfloat16)
        _gpu(k_norm, "k_norm", torch.bfloat16)
        _gpu(positions, "positions", torch.int64)
        _gpu(slots, "slots", torch.int64)
        _gpu(cos_sin, "cos_sin", torch.float32)
        _check(positions.numel() == m and slots.numel() == m, "positions/slots must have M entries")
        self._call("sid_rmsnorm_qkv_post", src.data_ptr(), f32, norm_w.data_ptr(), float(eps),
                   w.data_ptr(), m, hidden, hq, hkv, d, q_norm.data_ptr(), k_norm.data_ptr(),
                   positions.data_ptr(), cos_sin.data_ptr(), cos_sin.shape[0], slots.data_ptr(),
                   q_out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), k_cache.shape[0],
                   _stream(q_out))

    def pack_decode_weight(self, w, packed, gate_up: bool) -> None:
        """packed <- w [N, K] in the fragment-packed order of the decode-chain kernels."""
        _gpu(w, "weight", torch.bfloat16)
        _gpu(packed, "packed", torch.bfloat16)
        _check(w.dim() == 2 and packed.shape == w.shape, "packed must have the weight's shape")
        self._call("sid_pack_decode_weight", w.data_ptr(), packed.data_ptr(), w.shape[0],
                   w.shape[1], int(gate_up), _stream(packed))

    def rmsnorm_f32(self, x, w, out, eps: float) -> None:
        """out <- bf16(rmsnorm(x) * w) for fp32 rows x (rmsnorm's bits)."""
        _gpu(x, "x", torch.float32)
        _gpu(w, "weight", torch.bfloat16)
        _gpu(out, "out", torch.bfloat16)
        _check(x.dim() == 2 and out.shape == x.shape and w.numel() == x.shape[1], "rmsnorm_f32 shapes")
        self._call("sid_rmsnorm_f32", x.data_ptr(), w.data_ptr(), out.data_ptr(), x.shape[0],
                   x.shape[1], float(eps), _stream(out))

    def linear_silu_mul(self, x, w, out) -> None:
        _gpu(x, "x", torch.bfloat16)
        _gpu(w, "weight", torch.bfloat16)
        _gpu(out, "out", torch.bfloat16)
        _check(x.dim() == 2 and w.dim() == 2 and w.shape[1] == x.shape[1], "x / weight shapes")
        _check(w.shape[0] % 2 == 0 and tuple(out.shape) == (x.shape[0], w.shape[0] // 2),
               "linear_silu_mul: out must be [M, N/2]")
        self._call("sid_linear_silu_mul", x.data_ptr(), w.data_ptr(), out.data_ptr(), x.shape[0],
                   x.shape[1], w.shape[0] // 2, _stream(out))

    def silu_mul(self, gate_up, out) -> None:
        _gpu(gate_up, "gate_up", torch.bfloat16)
        _gpu(out, "out", torch.bfloat16)
        t, two_i = gate_up.shape
        _check(two_i % 2 == 0 and tuple(out.shape) == (t, two_i // 2), "silu_mul shape mismatch")
        self._call("sid_silu_mul", gate_up.data_ptr(), out.data_ptr(), t, two_i // 2, _stream(out))

    def gather_rows(self, table, idx, out) -> None:
        _gpu(table, "table", torch.bfloat16)
        _gpu(idx, "indices", torch.int64)
        _gpu(out, "out", torch.bfloat16)
        _check(out.shape[0] == idx.numel() and out.shape[1:] == table.shape[1:],
               "gather_rows shape mismatch")
        row = table[0].numel() if table.shape[0] > 0 else out[0].numel()
        self._call("sid_gather_rows", table.data_ptr(), idx.data_ptr(), out.data_ptr(),
                   idx.numel(), row, table.shape[0], _stream(out))

    def argmax_rows(self, logits, out) -> None:
        _check(logits.is_cuda and logits.dtype == torch.float32 and logits.dim() == 2
               and logits.stride(1) == 1, "logits must be 2-D fp32 on the GPU, unit column stride")
        _gpu(out, "out", torch.int64)
        _check(out.numel() == logits.shape[0], "out must have one entry per row")
        self._call("sid_argmax_rows", logits.data_ptr(), logits.stride(0), out.data_ptr(),
                   logits.shape[0], logits.shape[1], _stream(out))

    def sample_rows(self, logits, temperatures, top_ks, top_ps, seeds, positions, out) -> None:
        _check(logits.is_cuda and logits.dtype == torch.float32 and logits.dim() == 2
               and logits.stride(1) == 1, "logits must be 2-D fp32 on the GPU, unit column stride")
        r, v = logits.shape
        for name, t, dt in (("temperatures", temperatures, torch.float32),
                            ("top_ks", top_ks, torch.int64), ("top_ps", top_ps, torch.float32),
                            ("seeds", seeds, torch.int64), ("positions", positions, torch.int64),
                            ("out", out, torch.int64)):
            _gpu(t, name, dt)
            _check(t.numel() == r, f"{name} must have one entry per row")
        if r == 0:
            return
        ws = torch.empty(int(self.lib.sid_sample_workspace_bytes(r, v)), dtype=torch.uint8,
                         device=logits.device)
        self._call("sid_sample_rows", logits.data_ptr(), logits.stride(0), temperatures.data_ptr(),
                   top_ks.data_ptr(), top_ps.data_ptr(), seeds.data_ptr(), positions.data_ptr(),
                   r, v, ws.data_ptr(), ws.numel(), out.data_ptr(), _stream(logits))

    def build_paged_decode_indices(self, block_tables, page_size: int, rows, new_slots,
                                   kv_indptr, kv_indices) -> None:
        _gpu(block_tables, "block_tables", torch.int32)
        _check(block_tables.dim() == 2, "block_tables must be [rows, max_pages]")
        _gpu(rows, "rows", torch.int64)
        _gpu(new_slots, "new_slots", torch.int64)
        _check(new_slots.numel() == rows.numel(), "new_slots must have B entries")
        _gpu(kv_indptr, "kv_indptr", torch.int32)
        _gpu(kv_indices, "kv_indices", torch.int32)
        _check(kv_indptr.numel() == rows.numel() + 1, "kv_indptr must have B+1 entries")
        self._call("sid_build_paged_decode_indices", block_tables.data_ptr(),
                   block_tables.shape[1], block_tables.shape[0], int(page_size), rows.data_ptr(),
                   new_slots.data_ptr(), kv_indptr.data_ptr(), kv_indices.data_ptr(),
                   rows.numel(), _stream(rows))
