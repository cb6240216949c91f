"""Python binding of libgemma4_kv.so, the MI355X build of gemma.c's KV-cache
path (paged K/V append, split-K decode attention, prefill-chunk attention).

This module is a thin ctypes layer over the C-ABI declared in include/*.h; it
mirrors the reference's C++ entry points (same names, argument order and
hipError_t return codes) so tests read like the reference's own tests.
Device buffers are torch tensors (PyTorch supplies device memory and the
stream); nothing here computes on the host. If the shared library is missing
the import of any entry point raises: there is no fallback path.
"""
from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Optional

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libgemma4_kv.so"

HIP_SUCCESS = 0
HIP_ERROR_INVALID_VALUE = 1

QUERY_HEADS = 16


class Gemma4KvCacheConfig(ctypes.Structure):
    """Same 8 x int32 layout as the reference struct (src/gemma4_kv_cache.cuh:9-18)."""

    _fields_ = [
        ("num_layers", ctypes.c_int32),
        ("num_pages", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("max_pages_per_seq", ctypes.c_int32),
        ("batch_size", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("window_size", ctypes.c_int32),
    ]

    def as_tuple(self):
        return tuple(getattr(self, f) for f, _ in self._fields_)

    def __repr__(self) -> str:
        return "Gemma4KvCacheConfig(%s)" % ", ".join(
            f"{f}={getattr(self, f)}" for f, _ in self._fields_)


def make_config(num_layers, num_pages, page_size, max_pages_per_seq, batch_size,
                num_heads, head_dim, window_size) -> Gemma4KvCacheConfig:
    return Gemma4KvCacheConfig(num_layers, num_pages, page_size, max_pages_per_seq,
                               batch_size, num_heads, head_dim, window_size)


class HipError(RuntimeError):
    def __init__(self, code: int, what: str):
        super().__init__(f"{what} returned hipError_t {code}")
        self.code = code


_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_F32 = ctypes.c_float
_CFG = Gemma4KvCacheConfig

# name -> (restype, argtypes); every symbol include/*.h declares with C linkage.
SIGNATURES = {
    "gemma4_kv_cache_make_config": (_CFG, [ctypes.c_bool, _I32, _I32, _I32]),
    "gemma4_kv_cache_layer_index": (_I32, [_I32, ctypes.c_bool]),
    "gemma4_kv_cache_ensure_page_ptr": (_I32, [_P, _P, _I64, ctypes.POINTER(_CFG), _I32, _I32]),
    "gemma4_kv_cache_ensure_range_ptr": (_I32, [_P, _P, _I64, ctypes.POINTER(_CFG), _I32, _I32, _I32]),
    "gemma4_kv_cache_write_bf16": (_I32, [_P, _P, _CFG, _P, _P, _P, _I32, _I32, _P, _P, _P]),
    "gemma4_kv_cache_write_prefill_bf16": (_I32, [_P, _P, _CFG, _P, _P, _P, _I32, _I32, _I32, _P, _P, _P]),
    "gemma4_flash_attention_decode_paged_bf16": (
        _I32, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _CFG, _I32, _F32, _I32, _I32, _I32, _P]),
    "gemma4_flash_attention_append_decode_paged_bf16": (
        _I32, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _CFG, _I32, _F32, _I32, _I32, _I32, _P]),
    "gemma4_flash_attention_decode_split_paged_bf16": (
        _I32, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _CFG, _I32, _F32, _I32, _I32, _I32, _P]),
    "gemma4_flash_attention_decode_combine_bf16": (
        _I32, [_P, _P, _P, _P, _P, _CFG, _I32, _I32, _I32, _P]),
    "gemma4_flash_attention_prefill_chunk_paged_bf16": (
        _I32, [_P, _P, _P, _P, _P, _P, _P, _P, _CFG, _I32, _I32, _I32, _F32, _P]),
    "gemma4_flash_attention_prefill_chunk_workspace_bytes": (ctypes.c_size_t, [_I32, _I32, _CFG]),
    "gemma4_flash_attention_prefill_chunk_paged_bf16_ws": (
        _I32, [_P, _P, _P, _P, _P, _P, _P, _P, _CFG, _I32, _I32, _I32, _F32, _P, ctypes.c_size_t, _P]),
    "gemma4_flash_attention_sliding_fwd_bf16_norm_rope": (
        _I32, [_P] * 12 + [_I32, _I32, _I32, _I32, _F32, _P]),
    "gemma4_flash_attention_global_fwd_bf16_norm_rope": (
        _I32, [_P] * 11 + [_I32, _I32, _I32, _F32, _P]),
    "gemma4_flash_attention_prep_append_decode_paged_bf16": (
        _I32, [_P] * 17 + [_CFG, _I32, _F32, _I32, _I32, _I32, _P]),
    "gemma4_attention_o_projection_post_norm_bf16": (_I32, [_P] * 7 + [_I32, _I32, _P]),
    "gemma4_runtime_create": (_I32, [ctypes.POINTER(_P), _I32, _I32, _I32, _P]),
    "gemma4_runtime_destroy": (None, [_P]),
    "gemma4_runtime_prefill": (_I32, [_P, _I32, _P]),
    "gemma4_runtime_decode_step": (_I32, [_P, _P]),
    "gemma4_runtime_decode_step_device": (_I32, [_P, _P]),
    "gemma4_runtime_sync_host_state": (_I32, [_P, _P]),
    "gemma4_runtime_get_device_step_status": (_I32, [_P, ctypes.POINTER(_I32)]),
    "gemma4_runtime_get_config": (_I32, [_P, _I32, ctypes.POINTER(_CFG)]),
    "gemma4_runtime_get_scalars": (_I32, [_P, ctypes.POINTER(_I32)]),
    "gemma4_runtime_get_host_vector": (_I32, [_P, _I32, _P, _I64, ctypes.POINTER(_I64)]),
    "gemma4_runtime_set_host_seq_lengths": (_I32, [_P, _P, _I64]),
    "gemma4_runtime_device_ptr": (_P, [_P, _I32]),
    "gemma4_decode_split_plan": (_I32, [_CFG, _I32, _I32, _I32, ctypes.POINTER(_I32), ctypes.POINTER(_I32)]),
    "gemma4_decode_prep_append_bf16": (
        _I32, [_P, _P, _P, _CFG, _P, _P, _I32, _P, _P, _P, _P, _P, _P, _P, _I32, _P]),
    "gemma4_decode_step_workspace_bytes": (ctypes.c_size_t, [_I32]),
    "gemma4_decode_step_workspace_init": (_I32, [_P, ctypes.c_size_t, _I32, _P]),
    "gemma4_decode_step_status": (_I32, [_P, ctypes.POINTER(_I32)]),
    "gemma4_decode_step_status_async": (_I32, [_P, _P, _P]),
    "gemma4_flash_attention_append_decode_paged_bf16_noalloc": (
        _I32, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _CFG, _I32, _F32, _I32, _I32, _I32, _P]),
    "gemma4_decode_step_inject_stall": (_I32, [_P, _I32, ctypes.c_uint32, _P]),
    "gemma4_decode_step_set_cooperative": (_I32, [_I32]),
    "gemma4_decode_step_layers_prep_bf16": (
        _I32, [_P, _P, _P, _P, _P, _P, _P, _CFG, _P, _P, _P, _CFG, _P, _P, _P, _P, _P, _P, _P, _P,
               _I32, _I32, _F32, _I32, _P, ctypes.c_size_t, _P]),
    "gemma4_decode_walk_bf16": (
        _I32, [_P] * 7 + [_CFG, _I32, _P, _P, _I32, _F32, _I32, _P, ctypes.c_size_t, _P]),
    "gemma4_runtime_decode_walk": (_I32, [_P, _I32, _P]),
    "gemma4_decode_step_layers_bf16": (
        _I32, [_P, _P, _P, _P, _P, _P, _P, _CFG, _P, _P, _P, _CFG, _P, _P, _I32, _I32, _F32,
               _I32, _P, ctypes.c_size_t, _P]),
}

_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    """Load the in-tree shared library (after torch, so both share one HIP runtime)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is not built; run gemma_kv.build.build() (or __graft_entry__.build())")
    try:
        import torch  # noqa: F401  (loads the HIP runtime the library binds to)
    except ImportError:
        pass
    handle = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    _lib = handle
    return handle


def ptr(x) -> int:
    """Device/host address of a tensor, an int, or None (null)."""
    if x is None:
        return 0
    if isinstance(x, int):
        return x
    return x.data_ptr()


def stream_handle(stream=None) -> int:
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def check(code: int, what: str = "call") -> None:
    if code != HIP_SUCCESS:
        raise HipError(code, what)


# ---- host helpers (no device work) ---------------------------------------

def kv_cache_make_config(global_cache: bool, num_pages: int, page_size: int,
                         max_pages_per_seq: int) -> Gemma4KvCacheConfig:
    return lib().gemma4_kv_cache_make_config(bool(global_cache), num_pages, page_size,
                                             max_pages_per_seq)


def kv_cache_layer_index(model_layer: int, global_cache: bool) -> int:
    return lib().gemma4_kv_cache_layer_index(model_layer, bool(global_cache))


def kv_cache_ensure_page(page_table, slot_logical_pages, config, batch, position) -> int:
    """page_table / slot_logical_pages: int32 numpy arrays, mutated in place."""
    assert page_table.dtype.name == "int32" and slot_logical_pages.dtype.name == "int32"
    n = min(page_table.size, slot_logical_pages.size)
    return lib().gemma4_kv_cache_ensure_page_ptr(
        page_table.ctypes.data, slot_logical_pages.ctypes.data, n,
        ctypes.byref(config), batch, position)


def kv_cache_ensure_range(page_table, slot_logical_pages, config, batch,
                          first_position, token_count) -> int:
    assert page_table.dtype.name == "int32" and slot_logical_pages.dtype.name == "int32"
    n = min(page_table.size, slot_logical_pages.size)
    return lib().gemma4_kv_cache_ensure_range_ptr(
        page_table.ctypes.data, slot_logical_pages.ctypes.data, n,
        ctypes.byref(config), batch, first_position, token_count)


def decode_split_plan(config, batch_count: int, max_live_keys: int,
                      target_workgroups: int = 0):
    s = _I32()
    n = _I32()
    check(lib().gemma4_decode_split_plan(config, batch_count, max_live_keys,
                                         target_workgroups, ctypes.byref(s),
                                         ctypes.byref(n)), "gemma4_decode_split_plan")
    return s.value, n.value


# ---- device entry points (return hipError_t codes, like the reference) ----

def kv_cache_write_bf16(cache_k, cache_v, config, page_table, token_batch,
                        token_position, token_count, layer, k, v, stream=None) -> int:
    return lib().gemma4_kv_cache_write_bf16(
        ptr(cache_k), ptr(cache_v), config, ptr(page_table), ptr(token_batch),
        ptr(token_position), token_count, layer, ptr(k), ptr(v), stream_handle(stream))


def kv_cache_write_prefill_bf16(cache_k, cache_v, config, page_table, token_batch,
                                token_position, batch_size, seq_len, layer, k, v,
                                stream=None) -> int:
    return lib().gemma4_kv_cache_write_prefill_bf16(
        ptr(cache_k), ptr(cache_v), config, ptr(page_table), ptr(token_batch),
        ptr(token_position), batch_size, seq_len, layer, ptr(k), ptr(v),
        stream_handle(stream))


def flash_attention_decode_paged_bf16(out, partial_m, partial_l, partial_acc, q,
                                      cache_k, cache_v, page_table, seq_lengths,
                                      config, layer, softmax_scale, split_size,
                                      num_splits, batch_count, stream=None) -> int:
    return lib().gemma4_flash_attention_decode_paged_bf16(
        ptr(out), ptr(partial_m), ptr(partial_l), ptr(partial_acc), ptr(q),
        ptr(cache_k), ptr(cache_v), ptr(page_table), ptr(seq_lengths), config,
        layer, softmax_scale, split_size, num_splits, batch_count,
        stream_handle(stream))


def flash_attention_append_decode_paged_bf16(out, partial_m, partial_l, partial_acc,
                                             q, cache_k, cache_v, page_table,
                                             seq_lengths, token_position, k, v,
                                             config, layer, softmax_scale,
                                             split_size, num_splits, batch_count,
                                             stream=None, split_counters=None) -> int:
    return lib().gemma4_flash_attention_append_decode_paged_bf16(
        ptr(out), ptr(partial_m), ptr(partial_l), ptr(partial_acc), ptr(q),
        ptr(cache_k), ptr(cache_v), ptr(page_table), ptr(seq_lengths),
        ptr(token_position), ptr(k), ptr(v), ptr(split_counters), config, layer,
        softmax_scale,
        split_size, num_splits, batch_count, stream_handle(stream))


def flash_attention_append_decode_paged_bf16_noalloc(out, q, cache_k, cache_v, page_table,
                                                     seq_lengths, token_position, k, v, config,
                                                     layer, softmax_scale, split_size,
                                                     num_splits, batch_count,
                                                     stream=None) -> int:
    return lib().gemma4_flash_attention_append_decode_paged_bf16_noalloc(
        ptr(out), ptr(q), ptr(cache_k), ptr(cache_v), ptr(page_table), ptr(seq_lengths),
        ptr(token_position), ptr(k), ptr(v), config, layer, softmax_scale, split_size,
        num_splits, batch_count, stream_handle(stream))


def flash_attention_decode_split_paged_bf16(out, partial_m, partial_l, partial_acc, q,
                                            cache_k, cache_v, page_table, seq_lengths,
                                            token_position, k, v, config, layer,
                                            softmax_scale, split_size, num_splits,
                                            batch_count, stream=None) -> int:
    return lib().gemma4_flash_attention_decode_split_paged_bf16(
        ptr(out), ptr(partial_m), ptr(partial_l), ptr(partial_acc), ptr(q),
        ptr(cache_k), ptr(cache_v), ptr(page_table), ptr(seq_lengths),
        ptr(token_position), ptr(k), ptr(v), config, layer, softmax_scale,
        split_size, num_splits, batch_count, stream_handle(stream))


def flash_attention_decode_combine_bf16(out, partial_m, partial_l, partial_acc,
                                        seq_lengths, config, split_size, num_splits,
                                        batch_count, stream=None) -> int:
    return lib().gemma4_flash_attention_decode_combine_bf16(
        ptr(out), ptr(partial_m), ptr(partial_l), ptr(partial_acc), ptr(seq_lengths),
        config, split_size, num_splits, batch_count, stream_handle(stream))


def decode_prep_append_bf16(q_prepared, cache_k, cache_v, config, page_table, token_position,
                            layer, q, k, v, q_norm_weight, k_norm_weight, cos, sin,
                            batch_count, stream=None) -> int:
    return lib().gemma4_decode_prep_append_bf16(
        ptr(q_prepared), ptr(cache_k), ptr(cache_v), config, ptr(page_table),
        ptr(token_position), layer, ptr(q), ptr(k), ptr(v), ptr(q_norm_weight),
        ptr(k_norm_weight), ptr(cos), ptr(sin), batch_count, stream_handle(stream))


def decode_step_workspace_bytes(batch_count: int) -> int:
    return lib().gemma4_decode_step_workspace_bytes(batch_count)


def decode_step_workspace_init(workspace, batch_count: int, stream=None) -> int:
    return lib().gemma4_decode_step_workspace_init(
        ptr(workspace), workspace.numel() * workspace.element_size(), batch_count,
        stream_handle(stream))


def decode_step_status(workspace) -> int:
    st = _I32()
    check(lib().gemma4_decode_step_status(ptr(workspace), ctypes.byref(st)),
          "gemma4_decode_step_status")
    return st.value


def decode_step_status_async(workspace, status, stream=None) -> int:
    """Stream-ordered copy of the step status word into `status` (a device
    or pinned-host int32 tensor)."""
    return lib().gemma4_decode_step_status_async(ptr(workspace), ptr(status),
                                                 stream_handle(stream))


def decode_step_set_cooperative(enable: bool) -> int:
    return lib().gemma4_decode_step_set_cooperative(1 if enable else 0)


def decode_step_inject_stall(workspace, layer: int, limit_ticks: int, stream=None) -> int:
    return lib().gemma4_decode_step_inject_stall(ptr(workspace), layer, limit_ticks,
                                                 stream_handle(stream))


def decode_step_layers_bf16(out, q, k, v, sliding_k, sliding_v, sliding_page_table,
                            sliding_config, global_k, global_v, global_page_table,
                            global_config, seq_lengths, token_position, first_layer,
                            layer_count, softmax_scale, batch_count, workspace,
                            stream=None) -> int:
    return lib().gemma4_decode_step_layers_bf16(
        ptr(out), ptr(q), ptr(k), ptr(v), ptr(sliding_k), ptr(sliding_v),
        ptr(sliding_page_table), sliding_config, ptr(global_k), ptr(global_v),
        ptr(global_page_table), global_config, ptr(seq_lengths), ptr(token_position),
        first_layer, layer_count, softmax_scale, batch_count, ptr(workspace),
        workspace.numel() * workspace.element_size(), stream_handle(stream))


def decode_step_layers_prep_bf16(out, q, k, v, sliding_k, sliding_v, sliding_page_table,
                                 sliding_config, global_k, global_v, global_page_table,
                                 global_config, seq_lengths, token_position, q_norm_weight,
                                 k_norm_weight, sliding_cos, sliding_sin, global_cos, global_sin,
                                 first_layer, layer_count, softmax_scale, batch_count, workspace,
                                 stream=None) -> int:
    return lib().gemma4_decode_step_layers_prep_bf16(
        ptr(out), ptr(q), ptr(k), ptr(v), ptr(sliding_k), ptr(sliding_v),
        ptr(sliding_page_table), sliding_config, ptr(global_k), ptr(global_v),
        ptr(global_page_table), global_config, ptr(seq_lengths), ptr(token_position),
        ptr(q_norm_weight), ptr(k_norm_weight), ptr(sliding_cos), ptr(sliding_sin),
        ptr(global_cos), ptr(global_sin), first_layer, layer_count, softmax_scale, batch_count,
        ptr(workspace), workspace.numel() * workspace.element_size(), stream_handle(stream))


def decode_walk_bf16(out, q, k, v, cache_k, cache_v, page_table, config, layer,
                     seq_lengths, token_position, steps, softmax_scale, batch_count,
                     workspace, stream=None) -> int:
    return lib().gemma4_decode_walk_bf16(
        ptr(out), ptr(q), ptr(k), ptr(v), ptr(cache_k), ptr(cache_v), ptr(page_table), config,
        layer, ptr(seq_lengths), ptr(token_position), steps, softmax_scale, batch_count,
        ptr(workspace), workspace.numel() * workspace.element_size(), stream_handle(stream))


class Runtime:
    """Owner of a Gemma4RuntimeState (caches, page tables, token metadata),
    mirroring src/gemma4_runtime.cuh through the opaque-handle C-ABI."""

    HOST = {"sliding_page_table": 0, "global_page_table": 1, "sliding_slot_logical_pages": 2,
            "global_slot_logical_pages": 3, "seq_lengths": 4, "token_batch": 5,
            "token_position": 6}
    DEVICE = {"sliding_cache_k": 0, "sliding_cache_v": 1, "global_cache_k": 2,
              "global_cache_v": 3, "sliding_page_table": 4, "global_page_table": 5,
              "seq_lengths": 6, "token_batch": 7, "token_position": 8, "sliding_cos": 9,
              "sliding_sin": 10, "global_cos": 11, "global_sin": 12,
              "sliding_slot_logical_pages": 13, "global_slot_logical_pages": 14}

    def __init__(self, batch_size, max_seq_len, page_size, stream=None):
        self._h = ctypes.c_void_p()
        self.init_code = lib().gemma4_runtime_create(ctypes.byref(self._h), batch_size,
                                                     max_seq_len, page_size, stream_handle(stream))

    def close(self):
        if self._h:
            lib().gemma4_runtime_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def prepare_prefill(self, seq_len, stream=None) -> int:
        return lib().gemma4_runtime_prefill(self._h, seq_len, stream_handle(stream))

    def prepare_decode_step(self, stream=None) -> int:
        return lib().gemma4_runtime_decode_step(self._h, stream_handle(stream))

    def prepare_decode_step_device(self, stream=None) -> int:
        return lib().gemma4_runtime_decode_step_device(self._h, stream_handle(stream))

    def prepare_decode_walk(self, steps, stream=None) -> int:
        return lib().gemma4_runtime_decode_walk(self._h, steps, stream_handle(stream))

    def sync_host(self, stream=None) -> int:
        return lib().gemma4_runtime_sync_host_state(self._h, stream_handle(stream))

    def device_step_status(self) -> int:
        out = _I32()
        check(lib().gemma4_runtime_get_device_step_status(self._h, ctypes.byref(out)))
        return out.value

    def config(self, global_cache: bool) -> Gemma4KvCacheConfig:
        c = Gemma4KvCacheConfig()
        check(lib().gemma4_runtime_get_config(self._h, int(global_cache), ctypes.byref(c)))
        return c

    def scalars(self):
        out = (_I32 * 4)()
        check(lib().gemma4_runtime_get_scalars(self._h, out))
        return dict(zip(("batch_size", "max_seq_len", "page_size", "token_count"), list(out)))

    def host(self, name):
        import numpy as np
        size = _I64()
        check(lib().gemma4_runtime_get_host_vector(self._h, self.HOST[name], None, 0,
                                                   ctypes.byref(size)))
        arr = np.zeros(size.value, dtype=np.int32)
        check(lib().gemma4_runtime_get_host_vector(self._h, self.HOST[name], arr.ctypes.data,
                                                   arr.size, ctypes.byref(size)))
        return arr

    def set_host_seq_lengths(self, values):
        import numpy as np
        arr = np.ascontiguousarray(values, dtype=np.int32)
        check(lib().gemma4_runtime_set_host_seq_lengths(self._h, arr.ctypes.data, arr.size))

    def device_ptr(self, name) -> int:
        return lib().gemma4_runtime_device_ptr(self._h, self.DEVICE[name]) or 0


def flash_attention_sliding_fwd_bf16_norm_rope(out, q_prepared, k_prepared, v_prepared, q, k, v,
                                               q_norm_weight, k_norm_weight, cos, sin,
                                               token_position, batch_size, seqlen_q, seqlen_k,
                                               window_size, softmax_scale, stream=None) -> int:
    return lib().gemma4_flash_attention_sliding_fwd_bf16_norm_rope(
        ptr(out), ptr(q_prepared), ptr(k_prepared), ptr(v_prepared), ptr(q), ptr(k), ptr(v),
        ptr(q_norm_weight), ptr(k_norm_weight), ptr(cos), ptr(sin), ptr(token_position),
        batch_size, seqlen_q, seqlen_k, window_size, softmax_scale, stream_handle(stream))


def flash_attention_global_fwd_bf16_norm_rope(out, q_prepared, k_prepared, v_prepared, q, k,
                                              q_norm_weight, k_norm_weight, cos, sin,
                                              token_position, batch_size, seqlen_q, seqlen_k,
                                              softmax_scale, stream=None) -> int:
    return lib().gemma4_flash_attention_global_fwd_bf16_norm_rope(
        ptr(out), ptr(q_prepared), ptr(k_prepared), ptr(v_prepared), ptr(q), ptr(k),
        ptr(q_norm_weight), ptr(k_norm_weight), ptr(cos), ptr(sin), ptr(token_position),
        batch_size, seqlen_q, seqlen_k, softmax_scale, stream_handle(stream))


def flash_attention_prep_append_decode_paged_bf16(out, partial_m, partial_l, partial_acc, q,
                                                  cache_k, cache_v, page_table, seq_lengths,
                                                  token_position, k, v, q_norm_weight,
                                                  k_norm_weight, cos, sin, config, layer,
                                                  softmax_scale, split_size, num_splits,
                                                  batch_count, stream=None,
                                                  split_counters=None) -> int:
    return lib().gemma4_flash_attention_prep_append_decode_paged_bf16(
        ptr(out), ptr(partial_m), ptr(partial_l), ptr(partial_acc), ptr(q), ptr(cache_k),
        ptr(cache_v), ptr(page_table), ptr(seq_lengths), ptr(token_position), ptr(k), ptr(v),
        ptr(q_norm_weight), ptr(k_norm_weight), ptr(cos), ptr(sin), ptr(split_counters), config,
        layer, softmax_scale, split_size, num_splits, batch_count, stream_handle(stream))


def attention_o_projection_post_norm_bf16(residual_out, normed_out, ffn_residual, attention_out,
                                          o_proj_col_major, post_norm_weight, attention_x, rows,
                                          attention_width, stream=None) -> int:
    return lib().gemma4_attention_o_projection_post_norm_bf16(
        ptr(residual_out), ptr(normed_out), ptr(ffn_residual), ptr(attention_out),
        ptr(o_proj_col_major), ptr(post_norm_weight), ptr(attention_x), rows, attention_width,
        stream_handle(stream))


def flash_attention_prefill_chunk_workspace_bytes(batch_size, chunk_len, config) -> int:
    return lib().gemma4_flash_attention_prefill_chunk_workspace_bytes(batch_size, chunk_len, config)


def flash_attention_prefill_chunk_paged_bf16_ws(out, q, k, v, cache_k, cache_v, page_table,
                                                prior_lengths, config, layer, batch_size,
                                                chunk_len, softmax_scale, workspace,
                                                workspace_bytes, stream=None) -> int:
    return lib().gemma4_flash_attention_prefill_chunk_paged_bf16_ws(
        ptr(out), ptr(q), ptr(k), ptr(v), ptr(cache_k), ptr(cache_v), ptr(page_table),
        ptr(prior_lengths), config, layer, batch_size, chunk_len, softmax_scale, ptr(workspace),
        workspace_bytes, stream_handle(stream))


def flash_attention_prefill_chunk_paged_bf16(out, q, k, v, cache_k, cache_v, page_table,
                                             prior_lengths, config, layer, batch_size,
                                             chunk_len, softmax_scale, stream=None) -> int:
    return lib().gemma4_flash_attention_prefill_chunk_paged_bf16(
        ptr(out), ptr(q), ptr(k), ptr(v), ptr(cache_k), ptr(cache_v), ptr(page_table),
        ptr(prior_lengths), config, layer, batch_size, chunk_len, softmax_scale,
        stream_handle(stream))
