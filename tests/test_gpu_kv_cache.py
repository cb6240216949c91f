"""Bit-exact parity of the HIP K/V append (gemma4_kv_cache_write_bf16 and the
prefill-tail write) against the CPU oracle, plus the reference's own
invalid-row known answer (tests/test_kv_cache.cu:94-133)."""
import numpy as np
import pytest

import gemma_kv as gk
from kvtest import (cache_config, empty_bf16, fill_page_table, from_dev_bf16,
                    make_value, randn_bf16, ring_pages, to_dev)
from oracle import oracle

pytestmark = pytest.mark.gpu


def _cache_elems(cfg):
    num_layers, num_pages, page, _, _, heads, dim, _ = cfg
    return num_layers * num_pages * page * heads * dim


def test_invalid_page_row_writes_nothing(dev):
    # tests/test_kv_cache.cu:94-133: batch row 1 of a batch-1 cache is skipped.
    cfg = (1, 2, 4, 2, 1, 2, 16, 0)
    k = np.array([make_value(43000 + i) for i in range(2 * 16)], dtype=np.uint16)
    v = np.array([make_value(44000 + i) for i in range(2 * 16)], dtype=np.uint16)
    ck = empty_bf16(_cache_elems(cfg), dev)
    cv = empty_bf16(_cache_elems(cfg), dev)
    code = gk.kv_cache_write_bf16(ck, cv, gk.make_config(*cfg),
                                  to_dev(np.full(2, -1, np.int32), dev),
                                  to_dev(np.array([1], np.int32), dev),
                                  to_dev(np.array([0], np.int32), dev), 1, 0,
                                  to_dev(k, dev), to_dev(v, dev))
    gk.check(code)
    import torch
    torch.cuda.synchronize()
    assert not from_dev_bf16(ck).any() and not from_dev_bf16(cv).any()


@pytest.mark.parametrize("heads,dim,page,window,batch,tokens", [
    (8, 256, 1, 1024, 1, 1),        # decode append, sliding ring, page 1
    (8, 256, 64, 1024, 2, 37),      # paged sliding ring
    (8, 256, 64, 0, 3, 300),        # global cache
    (1, 512, 64, 0, 2, 129),        # reference global geometry
    (2, 16, 4, 0, 1, 9),            # reference test geometry
])
def test_append_matches_oracle(dev, heads, dim, page, window, batch, tokens):
    rng = np.random.default_rng(7 + tokens)
    max_pages = ring_pages(window, page) if window else (4096 + page - 1) // page
    cfg = cache_config(2, batch, page, max_pages, heads, dim, window)
    seq = rng.integers(1, 3000, size=batch)
    pt = fill_page_table(cfg, seq)
    pt[rng.integers(0, pt.size)] = -1  # one unmapped slot
    token_batch = rng.integers(-1, batch + 1, size=tokens).astype(np.int32)
    token_pos = rng.integers(-2, 3000, size=tokens).astype(np.int32)
    if tokens > 2:  # duplicate targets must resolve like the oracle (last writer wins is not relied on)
        token_batch[:] = np.arange(tokens) % max(batch, 1)
        token_pos[:] = np.arange(tokens) + 5
    k = randn_bf16(rng, (tokens, heads, dim))
    v = randn_bf16(rng, (tokens, heads, dim))
    ck0 = randn_bf16(rng, _cache_elems(cfg))
    cv0 = randn_bf16(rng, _cache_elems(cfg))
    exp_k, exp_v = ck0.copy(), cv0.copy()
    oracle.kv_cache_write(exp_k, exp_v, cfg, pt, token_batch, token_pos, 1, k, v)

    ck, cv = to_dev(ck0, dev), to_dev(cv0, dev)
    gk.check(gk.kv_cache_write_bf16(ck, cv, gk.make_config(*cfg), to_dev(pt, dev),
                                    to_dev(token_batch, dev), to_dev(token_pos, dev),
                                    tokens, 1, to_dev(k, dev), to_dev(v, dev)))
    assert np.array_equal(from_dev_bf16(ck), exp_k)
    assert np.array_equal(from_dev_bf16(cv), exp_v)


@pytest.mark.parametrize("window,seq_len", [(1024, 2048), (1024, 700), (0, 2048)])
def test_prefill_tail_write_matches_reference_policy(dev, window, seq_len):
    # src/gemma4_prefill_megakernel.cu:189-207: long sliding chunks keep only
    # the last window rows; the oracle replays the reference's per-batch calls.
    rng = np.random.default_rng(seq_len + window)
    heads, dim, page, batch = 8, 256, 1, 2
    max_pages = ring_pages(window, page) if window else seq_len
    cfg = cache_config(1, batch, page, max_pages, heads, dim, window)
    pt = np.full(batch * max_pages, -1, np.int32)
    slots = np.full_like(pt, -1)
    for b in range(batch):
        first = max(0, seq_len - window) if window else 0
        assert oracle.ensure_range(pt, slots, cfg, b, first, seq_len - first) == 0
    token_batch = np.repeat(np.arange(batch, dtype=np.int32), seq_len)
    token_pos = np.tile(np.arange(seq_len, dtype=np.int32), batch)
    k = randn_bf16(rng, (batch * seq_len, heads, dim))
    v = randn_bf16(rng, (batch * seq_len, heads, dim))
    exp_k = np.zeros(_cache_elems(cfg), np.uint16)
    exp_v = np.zeros_like(exp_k)
    if window and seq_len > window:
        for b in range(batch):
            r0 = b * seq_len + seq_len - window
            oracle.kv_cache_write(exp_k, exp_v, cfg, pt, token_batch[r0:r0 + window],
                                  token_pos[r0:r0 + window], 0, k[r0:r0 + window],
                                  v[r0:r0 + window])
    else:
        oracle.kv_cache_write(exp_k, exp_v, cfg, pt, token_batch, token_pos, 0, k, v)
    ck = empty_bf16(exp_k.size, dev)
    cv = empty_bf16(exp_k.size, dev)
    gk.check(gk.kv_cache_write_prefill_bf16(ck, cv, gk.make_config(*cfg), to_dev(pt, dev),
                                            to_dev(token_batch, dev), to_dev(token_pos, dev),
                                            batch, seq_len, 0, to_dev(k, dev), to_dev(v, dev)))
    assert np.array_equal(from_dev_bf16(ck), exp_k)
    assert np.array_equal(from_dev_bf16(cv), exp_v)


def test_append_error_convention(dev):
    cfg = gk.make_config(1, 2, 4, 2, 1, 2, 16, 0)
    buf = empty_bf16(1024, dev)
    idx = to_dev(np.zeros(4, np.int32), dev)
    # token_count == 0 succeeds without touching anything, even with nulls.
    assert gk.kv_cache_write_bf16(None, None, cfg, None, None, None, 0, 0, None, None) == 0
    assert gk.kv_cache_write_bf16(buf, buf, cfg, idx, idx, idx, -1, 0, buf, buf) == gk.HIP_ERROR_INVALID_VALUE
    assert gk.kv_cache_write_bf16(buf, buf, cfg, idx, idx, idx, 1, 1, buf, buf) == gk.HIP_ERROR_INVALID_VALUE
    assert gk.kv_cache_write_bf16(buf, None, cfg, idx, idx, idx, 1, 0, buf, buf) == gk.HIP_ERROR_INVALID_VALUE
    bad = gk.make_config(1, 2, 4, 2, 1, 2, 12, 0)  # head_dim not a multiple of 8
    assert gk.kv_cache_write_bf16(buf, buf, bad, idx, idx, idx, 1, 0, buf, buf) == gk.HIP_ERROR_INVALID_VALUE
