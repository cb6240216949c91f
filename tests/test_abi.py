"""The C-ABI library loads on a GPU-less host, exports every extern "C"
symbol include/*.h declares, and its host-only helpers (no device work)
agree with the reference semantics."""
import re
from pathlib import Path

import numpy as np
import pytest

import gemma_kv as gk
from oracle import oracle

REPO = Path(__file__).resolve().parent.parent


def declared_c_symbols():
    names = set()
    for h in (REPO / "include").glob("*.h"):
        text = h.read_text()
        # Only declarations inside extern "C" blocks are C-ABI symbols.
        for block in re.findall(r'extern "C" \{(.*?)\n\}', text, flags=re.S):
            block = re.sub(r"//.*", "", block)
            for m in re.finditer(r"\b(gemma4_\w+)\s*\(", block):
                names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    lib = gk.lib()
    names = declared_c_symbols()
    assert "gemma4_kv_cache_write_bf16" in names
    assert "gemma4_flash_attention_decode_paged_bf16" in names
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    # Every declared symbol has a binding signature in the Python mirror.
    assert names <= set(gk.SIGNATURES), sorted(names - set(gk.SIGNATURES))


def test_config_struct_layout():
    import ctypes
    assert ctypes.sizeof(gk.Gemma4KvCacheConfig) == 32
    assert [f for f, _ in gk.Gemma4KvCacheConfig._fields_] == [
        "num_layers", "num_pages", "page_size", "max_pages_per_seq", "batch_size",
        "num_heads", "head_dim", "window_size"]


@pytest.mark.parametrize("global_cache", [False, True])
def test_make_config_matches_oracle(global_cache):
    for args in [(2048, 1, 1024), (34, 64, 17), (128, 64, 64), (7, 3, 2)]:
        got = gk.kv_cache_make_config(global_cache, *args).as_tuple()
        assert got == oracle.make_config(global_cache, *args)


def test_layer_index_matches_oracle():
    for layer in range(-2, 50):
        for g in (False, True):
            assert gk.kv_cache_layer_index(layer, g) == oracle.layer_index(layer, g)
    # 5:1 cadence with the last layer global: 40 sliding + 8 global.
    assert sum(oracle.is_global_layer(l) for l in range(48)) == 8
    assert gk.kv_cache_layer_index(47, True) == 7


def test_ensure_page_ring_matches_oracle():
    rng = np.random.default_rng(3)
    for page, max_pages, batch in [(1, 1024, 2), (64, 17, 3), (4, 2, 1)]:
        cfg = (1, batch * max_pages, page, max_pages, batch, 8, 256, 1024)
        c = gk.make_config(*cfg)
        pt_a = np.full(batch * max_pages, -1, np.int32)
        sl_a = pt_a.copy()
        pt_b, sl_b = pt_a.copy(), sl_a.copy()
        pos = np.zeros(batch, np.int64)
        for _ in range(400):
            b = int(rng.integers(0, batch))
            step = int(rng.integers(-3, 90))  # occasional backwards (stale) use
            p = max(0, int(pos[b]) + step)
            pos[b] = max(pos[b], p)
            ra = gk.kv_cache_ensure_page(pt_a, sl_a, c, b, p)
            rb = oracle.ensure_page(pt_b, sl_b, cfg, b, p)
            assert ra == rb
            n = int(rng.integers(0, 200))
            ra = gk.kv_cache_ensure_range(pt_a, sl_a, c, b, p, n)
            rb = oracle.ensure_range(pt_b, sl_b, cfg, b, p, n)
            assert ra == rb
        assert np.array_equal(pt_a, pt_b) and np.array_equal(sl_a, sl_b)


def test_split_plan_fills_the_chip():
    c = gk.make_config(40, 1024, 1, 1024, 1, 8, 256, 1024)
    size, n = gk.decode_split_plan(c, 1, 1024)
    assert size * n >= 1024 and 8 * n >= 256
    # A 1024-key window at one sequence: one 16-key tile per workgroup (512
    # workgroups, two per CU).
    assert (size, n) == (16, 64)
    # An explicit target keeps whole 32-key chunks.
    size, n = gk.decode_split_plan(c, 1, 1024, 256)
    assert (size, n) == (32, 32)
    c = gk.make_config(8, 128, 64, 128, 1, 8, 256, 0)
    size, n = gk.decode_split_plan(c, 1, 8192)
    assert size * n >= 8192 and 8 * n >= 256
    size, n = gk.decode_split_plan(c, 64, 32768)
    assert size * n >= 32768
    # 1 x 512 (staged 16-key steps): 8193 keys as 171 splits of 48.
    c = gk.make_config(8, 129, 64, 129, 1, 1, 512, 0)
    assert gk.decode_split_plan(c, 1, 8193) == (48, 171)
