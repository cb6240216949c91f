"""numpy binding of the C oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker; never by the product library.
bf16 arrays are numpy uint16 bit patterns.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle.so"


class OracleKvCacheConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "num_layers", "num_pages", "page_size", "max_pages_per_seq", "batch_size",
        "num_heads", "head_dim", "window_size")]


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR), "liboracle.so"], check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        P = ctypes.c_void_p
        I = ctypes.c_int32
        F = ctypes.c_float
        C = ctypes.POINTER(OracleKvCacheConfig)
        sig = {
            "oracle_f32_to_bf16": (ctypes.c_uint16, [F]),
            "oracle_bf16_to_f32": (F, [ctypes.c_uint16]),
            "oracle_kv_cache_offset": (ctypes.c_int64, [C, I, I, I, I, I]),
            "oracle_kv_cache_make_config": (None, [C, I, I, I, I]),
            "oracle_is_global_layer": (I, [I]),
            "oracle_kv_cache_layer_index": (I, [I, I]),
            "oracle_kv_cache_ensure_page": (I, [P, P, C, I, I]),
            "oracle_kv_cache_ensure_range": (I, [P, P, C, I, I, I]),
            "oracle_sliding_pages_per_sequence": (I, [I, I]),
            "oracle_kv_cache_write": (None, [P, P, C, P, P, P, I, I, P, P]),
            "oracle_decode_attention": (None, [P, P, P, P, P, P, C, I, F, I, I]),
            "oracle_decode_split": (None, [P, P, P, P, P, P, P, P, C, I, F, I, I, I, I]),
            "oracle_decode_combine": (None, [P, P, P, P, P, C, I, I, I, I]),
            "oracle_prefill_attention": (None, [P, P, P, P, I, I, I, I, I, I, I, F]),
            "oracle_rms_scale": (F, [P, I, F]),
            "oracle_prep_head": (None, [P, P, P, P, P, I, I, F]),
            "oracle_fill_rope_tables": (None, [P, P, I, I, F, I]),
            "oracle_attention_o_projection": (None, [P, P, P, P, P, P, P, I, I, I, F]),
            "oracle_f32_to_bf16_array": (None, [P, P, ctypes.c_int64]),
            "oracle_bf16_to_f32_array": (None, [P, P, ctypes.c_int64]),
            "oracle_fill_normal_bf16": (None, [P, ctypes.c_int64, ctypes.c_uint64, F, I]),
            "oracle_time_decode_layer": (ctypes.c_double,
                                         [P, P, P, P, P, P, P, P, P, C, I, F, I, I, I]),
            "oracle_time_config1": (ctypes.c_double, [P, P, P, P, P, P, P, P, C, F, I, I, I]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(_lib, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


def cfg(c) -> OracleKvCacheConfig:
    """Accepts a tuple/sequence of 8 ints or any object with the 8 fields."""
    if hasattr(c, "num_layers"):
        vals = [getattr(c, n) for n, _ in OracleKvCacheConfig._fields_]
    else:
        vals = list(c)
    return OracleKvCacheConfig(*vals)


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def f32_to_bf16(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_bf16_array(_p(x), _p(out), x.size)
    return out


def bf16_to_f32(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.uint16)
    out = np.empty(x.shape, dtype=np.float32)
    lib().oracle_bf16_to_f32_array(_p(x), _p(out), x.size)
    return out


def kv_cache_offset(c, layer, page, page_offset, head, dim) -> int:
    cc = cfg(c)
    return lib().oracle_kv_cache_offset(ctypes.byref(cc), layer, page, page_offset, head, dim)


def make_config(global_cache, num_pages, page_size, max_pages_per_seq):
    cc = OracleKvCacheConfig()
    lib().oracle_kv_cache_make_config(ctypes.byref(cc), int(global_cache), num_pages,
                                      page_size, max_pages_per_seq)
    return tuple(getattr(cc, n) for n, _ in OracleKvCacheConfig._fields_)


def layer_index(model_layer, global_cache) -> int:
    return lib().oracle_kv_cache_layer_index(model_layer, int(global_cache))


def is_global_layer(layer) -> bool:
    return bool(lib().oracle_is_global_layer(layer))


def ensure_page(page_table, slot_logical, c, batch, position) -> int:
    cc = cfg(c)
    return lib().oracle_kv_cache_ensure_page(_p(page_table), _p(slot_logical),
                                             ctypes.byref(cc), batch, position)


def ensure_range(page_table, slot_logical, c, batch, first, count) -> int:
    cc = cfg(c)
    return lib().oracle_kv_cache_ensure_range(_p(page_table), _p(slot_logical),
                                              ctypes.byref(cc), batch, first, count)


def sliding_pages_per_sequence(max_seq_len, page_size) -> int:
    return lib().oracle_sliding_pages_per_sequence(max_seq_len, page_size)


def kv_cache_write(cache_k, cache_v, c, page_table, token_batch, token_position,
                   layer, k, v) -> None:
    cc = cfg(c)
    tb = np.ascontiguousarray(token_batch, dtype=np.int32)
    tp = np.ascontiguousarray(token_position, dtype=np.int32)
    lib().oracle_kv_cache_write(_p(cache_k), _p(cache_v), ctypes.byref(cc),
                                _p(np.ascontiguousarray(page_table, dtype=np.int32)),
                                _p(tb), _p(tp), tb.size, layer,
                                _p(np.ascontiguousarray(k)), _p(np.ascontiguousarray(v)))


def decode_attention(q, cache_k, cache_v, page_table, seq_lengths, c, layer, scale,
                     q_heads=16) -> np.ndarray:
    cc = cfg(c)
    q = np.ascontiguousarray(q, dtype=np.uint16)
    sl = np.ascontiguousarray(seq_lengths, dtype=np.int32)
    out = np.zeros(q.shape, dtype=np.uint16)
    lib().oracle_decode_attention(_p(out), _p(q), _p(cache_k), _p(cache_v),
                                  _p(np.ascontiguousarray(page_table, dtype=np.int32)),
                                  _p(sl), ctypes.byref(cc), layer, scale, sl.size, q_heads)
    return out


def decode_split(q, cache_k, cache_v, page_table, seq_lengths, c, layer, scale,
                 split_size, num_splits, q_heads=16):
    cc = cfg(c)
    q = np.ascontiguousarray(q, dtype=np.uint16)
    sl = np.ascontiguousarray(seq_lengths, dtype=np.int32)
    rows = sl.size * q_heads
    pm = np.full(rows * num_splits, np.nan, dtype=np.float32)
    pl = np.full(rows * num_splits, np.nan, dtype=np.float32)
    pa = np.full(rows * num_splits * cc.head_dim, np.nan, dtype=np.float32)
    lib().oracle_decode_split(_p(pm), _p(pl), _p(pa), _p(q), _p(cache_k), _p(cache_v),
                              _p(np.ascontiguousarray(page_table, dtype=np.int32)), _p(sl),
                              ctypes.byref(cc), layer, scale, split_size, num_splits,
                              sl.size, q_heads)
    return pm, pl, pa


def decode_combine(pm, pl, pa, seq_lengths, c, split_size, num_splits, q_heads=16):
    cc = cfg(c)
    sl = np.ascontiguousarray(seq_lengths, dtype=np.int32)
    out = np.zeros((sl.size, q_heads, cc.head_dim), dtype=np.uint16)
    lib().oracle_decode_combine(_p(out), _p(pm), _p(pl), _p(pa), _p(sl), ctypes.byref(cc),
                                split_size, num_splits, sl.size, q_heads)
    return out


def prefill_attention(q, k, v, seqlen_q, seqlen_k, q_heads, kv_heads, head_dim,
                      window, scale, batch=1) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    out = np.zeros(q.shape, dtype=np.uint16)
    lib().oracle_prefill_attention(_p(out), _p(q), _p(k), _p(v), batch, seqlen_q,
                                   seqlen_k, q_heads, kv_heads, head_dim, window, scale)
    return out


def rms_scale(values, eps=1e-6) -> float:
    v = np.ascontiguousarray(values, dtype=np.float32)
    return lib().oracle_rms_scale(_p(v), v.size, eps)


def prep_head(x, weight, cos_row, sin_row, rotary_dim, eps=1e-6) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.uint16)
    out = np.zeros_like(x)
    w = None if weight is None else np.ascontiguousarray(weight, dtype=np.uint16)
    c = None if cos_row is None else np.ascontiguousarray(cos_row, dtype=np.float32)
    s = None if sin_row is None else np.ascontiguousarray(sin_row, dtype=np.float32)
    lib().oracle_prep_head(_p(out), _p(x), 0 if w is None else _p(w),
                           0 if c is None else _p(c), 0 if s is None else _p(s),
                           x.size, rotary_dim, eps)
    return out


def fill_rope_tables(max_seq_len, rotary_half, theta, exponent_dim):
    cos = np.zeros(max_seq_len * rotary_half, dtype=np.float32)
    sin = np.zeros_like(cos)
    lib().oracle_fill_rope_tables(_p(cos), _p(sin), max_seq_len, rotary_half, theta,
                                  exponent_dim)
    return cos, sin


def attention_o_projection(attn, w_col_major, norm_weight, x, eps=1e-6):
    """attn [rows][width], w_col_major [hidden][width], norm_weight [hidden],
    x [rows][hidden] (bf16 bits) -> (residual_out, normed_out, ffn_residual)."""
    attn = np.ascontiguousarray(attn, dtype=np.uint16)
    w = np.ascontiguousarray(w_col_major, dtype=np.uint16)
    g = np.ascontiguousarray(norm_weight, dtype=np.uint16)
    x = np.ascontiguousarray(x, dtype=np.uint16)
    rows, width = attn.shape
    hidden = w.shape[0]
    assert w.shape == (hidden, width) and g.shape == (hidden,) and x.shape == (rows, hidden)
    outs = [np.zeros((rows, hidden), dtype=np.uint16) for _ in range(3)]
    lib().oracle_attention_o_projection(*(_p(o) for o in outs), _p(attn), _p(w), _p(g), _p(x),
                                        rows, width, hidden, eps)
    return tuple(outs)


# ---- CPU baseline timings (cpu_baseline.c) --------------------------------

def fill_normal_bf16(shape, seed, scale=1.0, threads=1) -> np.ndarray:
    """Seeded N(0,1)*scale bf16 array; values independent of `threads`."""
    out = np.empty(shape, dtype=np.uint16)
    lib().oracle_fill_normal_bf16(_p(out), out.size, seed, scale, threads)
    return out


def time_decode_layer(out, q, cache_k, cache_v, page_table, seq_lengths, token_position,
                      k_new, v_new, c, layer, scale, threads, q_heads=16) -> float:
    """Append + decode attention of one layer-step for len(seq_lengths)
    sequences, timed in C; writes `out` and the caches in place."""
    cc = cfg(c)
    sl = np.ascontiguousarray(seq_lengths, dtype=np.int32)
    tp = np.ascontiguousarray(token_position, dtype=np.int32)
    pt = np.ascontiguousarray(page_table, dtype=np.int32)
    return lib().oracle_time_decode_layer(_p(out), _p(q), _p(cache_k), _p(cache_v), _p(pt),
                                          _p(sl), _p(tp), _p(k_new), _p(v_new), ctypes.byref(cc),
                                          layer, scale, sl.size, q_heads, threads)


def time_config1(q, k, v, c, scale, threads, q_heads=16):
    """The config-1 loop (ensure_page, append, attend per step) from an empty
    ring, timed in C. Returns (seconds, out [steps][q_heads][head_dim],
    cache_k, cache_v, page_table)."""
    cc = cfg(c)
    steps = q.shape[0]
    rows = cc.num_layers * cc.num_pages * cc.page_size * cc.num_heads * cc.head_dim
    ck = np.zeros(rows, np.uint16)
    cv = np.zeros(rows, np.uint16)
    pt = np.full(cc.batch_size * cc.max_pages_per_seq, -1, np.int32)
    slots = np.full(cc.batch_size * cc.max_pages_per_seq, -1, np.int32)
    out = np.zeros((steps, q_heads, cc.head_dim), np.uint16)
    sec = lib().oracle_time_config1(_p(out), _p(np.ascontiguousarray(q)), _p(np.ascontiguousarray(k)),
                                    _p(np.ascontiguousarray(v)), _p(ck), _p(cv), _p(pt), _p(slots),
                                    ctypes.byref(cc), scale, steps, q_heads, threads)
    return sec, out, ck, cv, pt
