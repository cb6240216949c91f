"""Shared helpers for the KV-cache path tests: seeded bf16 inputs, cache
construction through the reference's ring bookkeeping, device transfer and
the reference's diff statistics (src/benches/gemma4_flash_attention_bench.cu:310-325)."""
from __future__ import annotations

import numpy as np

from oracle import oracle

# North-star tolerance for bf16 attention outputs against the fp32 reference.
MAX_ABS = 2e-2
MAX_REL = 1e-2


def randn_bf16(rng, shape, scale=1.0) -> np.ndarray:
    return oracle.f32_to_bf16(rng.standard_normal(shape, dtype=np.float32) * scale)


def make_value(seed: int) -> np.uint16:
    """Reference test generator (tests/test_kv_cache.cu:42-45)."""
    centered = ((seed * 37 + 17) % 257) - 128
    return oracle.f32_to_bf16(np.float32(centered) / np.float32(64.0))


def make_prefill_value(seed: int) -> np.uint16:
    """tests/test_flash_attention.cu:50-53"""
    centered = ((seed * 29 + 11) % 257) - 128
    return oracle.f32_to_bf16(np.float32(centered) / np.float32(512.0))


def diff_stats(a_bits: np.ndarray, b_bits: np.ndarray):
    a = oracle.bf16_to_f32(a_bits).astype(np.float32)
    b = oracle.bf16_to_f32(b_bits).astype(np.float32)
    diff = np.abs(a - b)
    denom = np.maximum(np.maximum(np.abs(a), np.abs(b)), 1.0)
    return float(diff.max(initial=0.0)), float((diff / denom).max(initial=0.0))


def assert_close(got_bits, exp_bits, what=""):
    max_abs, max_rel = diff_stats(got_bits, exp_bits)
    assert max_abs <= MAX_ABS and max_rel <= MAX_REL, (
        f"{what}: max_abs={max_abs:.4g} max_rel={max_rel:.4g}")
    return max_abs, max_rel


def cache_config(num_layers, batch, page_size, max_pages, heads, dim, window):
    return (num_layers, batch * max_pages, page_size, max_pages, batch, heads, dim, window)


def ring_pages(window: int, page_size: int) -> int:
    """Sliding ring slots per sequence (src/gemma4_runtime.cu:18-24 for a long max_seq)."""
    return (window + page_size - 1 + page_size - 1) // page_size


def fill_page_table(cfg, seq_lengths) -> np.ndarray:
    """Page table after every sequence's positions [0, len) were ensured, as
    gemma4_runtime_prepare_prefill + decode steps leave it."""
    num_layers, num_pages, page, max_pages, batch, heads, dim, window = cfg
    pt = np.full(batch * max_pages, -1, dtype=np.int32)
    slots = np.full(batch * max_pages, -1, dtype=np.int32)
    for b, n in enumerate(seq_lengths):
        if n > 0:
            assert oracle.ensure_range(pt, slots, cfg, b, 0, int(n)) == 0
    return pt


# ---- device transfer (torch supplies device memory) -----------------------

def to_dev(a: np.ndarray, dev):
    import torch
    if a.dtype == np.uint16:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def from_dev_bf16(t) -> np.ndarray:
    return t.cpu().numpy().view(np.uint16)


def empty_bf16(shape, dev):
    import torch
    return torch.zeros(shape, dtype=torch.int16, device=dev)


def torch_decode_reference(q_bits_t, cache_k_t, cache_v_t, page_table, seq_lengths,
                           cfg, layer, scale):
    """fp32 torch reference of paged decode attention on the GPU, for sizes the
    CPU oracle cannot cover in seconds. Inputs are int16 device tensors holding
    bf16 bits; returns fp32 [batch][16][dim]."""
    import torch
    num_layers, num_pages, page, max_pages, batch, heads, dim, window = cfg
    q = q_bits_t.view(torch.bfloat16).float()
    ck = cache_k_t.view(torch.bfloat16).view(-1, heads, dim)
    cv = cache_v_t.view(torch.bfloat16).view(-1, heads, dim)
    group = 16 // heads
    outs = []
    for b, n in enumerate(seq_lengths):
        n = int(n)
        first = max(0, n - window) if window > 0 else 0
        keys = torch.arange(first, n, device=q.device, dtype=torch.int64)
        if keys.numel() == 0:
            outs.append(torch.zeros(16, dim, device=q.device))
            continue
        lp = keys // page
        slot = lp % max_pages
        pt = torch.as_tensor(page_table, device=q.device, dtype=torch.int64)
        phys = pt[b * max_pages + slot]
        ok = (phys >= 0) & (phys < num_pages)
        rows = (layer * num_pages + phys) * page + (keys - lp * page)
        rows = rows[ok]
        k = ck[rows].float()  # [n, heads, dim]
        v = cv[rows].float()
        qb = q[b].view(heads, group, dim)
        s = torch.einsum("hgd,nhd->hgn", qb, k) * scale
        p = torch.softmax(s, dim=-1)
        o = torch.einsum("hgn,nhd->hgd", p, v).reshape(16, dim)
        outs.append(o)
    return torch.stack(outs)


def device_i16(ptr: int, count: int, dev):
    """Copy `count` int16 (bf16 bit patterns) from a raw device address that
    the library owns (e.g. a runtime cache) into a new tensor."""
    import ctypes
    import torch
    out = torch.empty(count, dtype=torch.int16, device=dev)
    hip = ctypes.CDLL("libamdhip64.so.7")  # the runtime torch already loaded (same soname)
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert hip.hipMemcpy(out.data_ptr(), ptr, count * 2, 3) == 0  # device to device
    torch.cuda.synchronize()
    return out
