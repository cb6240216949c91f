"""The allocation-free entry point
gemma4_flash_attention_append_decode_paged_bf16_noalloc against the entry
point it mirrors (gemma4_flash_attention_append_decode_paged_bf16 with
caller-allocated partials and the separate combine): the same kernels, so the
outputs and the appended caches must be bit-identical. Two calls in a row on
the library's shared scratch, the second with a smaller input (fewer
sequences, fewer splits, the other geometry), then a call past the scratch
limit, which must be refused before any launch."""
import math

import numpy as np
import pytest

import gemma_kv as gk
from kvtest import cache_config, fill_page_table, from_dev_bf16, randn_bf16, ring_pages, to_dev

pytestmark = pytest.mark.gpu

HIP_ERROR_OUT_OF_MEMORY = 2


def _case(rng, seq, heads, dim, window, page):
    batch = len(seq)
    max_pages = ring_pages(window, page) if window else (max(seq) + page - 1) // page
    cfg = cache_config(1, batch, page, max_pages, heads, dim, window)
    pt = fill_page_table(cfg, seq)
    rows = cfg[1] * page
    ck = randn_bf16(rng, (rows, heads, dim))
    cv = randn_bf16(rng, (rows, heads, dim))
    q = randn_bf16(rng, (batch, 16, dim))
    k = randn_bf16(rng, (batch, heads, dim))
    v = randn_bf16(rng, (batch, heads, dim))
    return cfg, pt, ck, cv, q, k, v


def _both(dev, cfg, pt, ck, cv, q, k, v, seq):
    import torch
    batch = len(seq)
    dim = cfg[6]
    conf = gk.make_config(*cfg)
    live = max(min(n, cfg[7]) if cfg[7] else n for n in seq)
    split, n = gk.decode_split_plan(conf, batch, live)
    d_seq = to_dev(np.asarray(seq, np.int32), dev)
    d_pos = to_dev(np.asarray([s - 1 for s in seq], np.int32), dev)
    d_pt, d_q, d_k, d_v = to_dev(pt, dev), to_dev(q, dev), to_dev(k, dev), to_dev(v, dev)
    ref_k, ref_v = to_dev(ck, dev), to_dev(cv, dev)
    got_k, got_v = to_dev(ck, dev), to_dev(cv, dev)
    ref_out = torch.zeros((batch, 16, dim), dtype=torch.int16, device=dev)
    got_out = torch.full((batch, 16, dim), 0x7fff, dtype=torch.int16, device=dev)
    pm = torch.empty(batch * 16 * n, device=dev)
    pl = torch.empty_like(pm)
    pa = torch.empty(batch * 16 * n * dim, device=dev)
    scale = 1 / math.sqrt(dim)
    gk.check(gk.flash_attention_append_decode_paged_bf16(
        ref_out, pm, pl, pa, d_q, ref_k, ref_v, d_pt, d_seq, d_pos, d_k, d_v, conf, 0, scale,
        split, n, batch), "workspace form")
    gk.check(gk.flash_attention_append_decode_paged_bf16_noalloc(
        got_out, d_q, got_k, got_v, d_pt, d_seq, d_pos, d_k, d_v, conf, 0, scale, split, n,
        batch), "noalloc form")
    torch.cuda.synchronize()
    assert n > 1  # the scratch is exercised
    assert torch.equal(got_out, ref_out)
    assert torch.equal(got_k, ref_k) and torch.equal(got_v, ref_v)
    assert from_dev_bf16(got_out).any()
    return n


def test_noalloc_matches_workspace_form_on_two_calls(dev):
    rng = np.random.default_rng(77)
    seq1 = [3000, 17, 1024, 700]
    print("noalloc: call 1 (4 sequences, 8x256 ring)", flush=True)
    n1 = _both(dev, *_case(rng, seq1, 8, 256, 1024, 16), seq1)
    seq2 = [300]
    print("noalloc: call 2 (1 sequence, 1x512 global)", flush=True)
    n2 = _both(dev, *_case(rng, seq2, 1, 512, 0, 64), seq2)
    assert 4 * n1 * 256 > n2 * 512  # the second call's partials are the smaller


def test_noalloc_single_split_writes_directly(dev):
    """num_splits == 1: no partials at all (the direct-output path), same
    result as the workspace form."""
    import torch
    rng = np.random.default_rng(5)
    seq = [40, 7]
    cfg, pt, ck, cv, q, k, v = _case(rng, seq, 8, 256, 0, 16)
    conf = gk.make_config(*cfg)
    d_seq = to_dev(np.asarray(seq, np.int32), dev)
    d_pos = to_dev(np.asarray([n - 1 for n in seq], np.int32), dev)
    d_pt, d_q, d_k, d_v = to_dev(pt, dev), to_dev(q, dev), to_dev(k, dev), to_dev(v, dev)
    outs = []
    for noalloc in (False, True):
        c_k, c_v = to_dev(ck, dev), to_dev(cv, dev)
        out = torch.zeros((2, 16, 256), dtype=torch.int16, device=dev)
        if noalloc:
            code = gk.flash_attention_append_decode_paged_bf16_noalloc(
                out, d_q, c_k, c_v, d_pt, d_seq, d_pos, d_k, d_v, conf, 0, 0.0625, 64, 1, 2)
        else:
            code = gk.flash_attention_append_decode_paged_bf16(
                out, None, None, None, d_q, c_k, c_v, d_pt, d_seq, d_pos, d_k, d_v, conf, 0,
                0.0625, 64, 1, 2)
        gk.check(code, "single split")
        torch.cuda.synchronize()
        outs.append((out, c_k, c_v))
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], outs[1][1]) and torch.equal(outs[0][2], outs[1][2])


def test_noalloc_allocates_no_device_memory(dev):
    """After a warm-up call (which looks up the scratch address once), a
    further call leaves the device's free memory unchanged."""
    import torch
    rng = np.random.default_rng(11)
    seq = [2000, 513]
    cfg, pt, ck, cv, q, k, v = _case(rng, seq, 8, 256, 0, 16)
    conf = gk.make_config(*cfg)
    split, n = gk.decode_split_plan(conf, len(seq), max(seq))
    assert n > 1
    d_seq = to_dev(np.asarray(seq, np.int32), dev)
    d_pos = to_dev(np.asarray([s - 1 for s in seq], np.int32), dev)
    d_pt, d_q, d_k, d_v = to_dev(pt, dev), to_dev(q, dev), to_dev(k, dev), to_dev(v, dev)
    c_k, c_v = to_dev(ck, dev), to_dev(cv, dev)
    out = torch.zeros((len(seq), 16, 256), dtype=torch.int16, device=dev)

    def call():
        gk.check(gk.flash_attention_append_decode_paged_bf16_noalloc(
            out, d_q, c_k, c_v, d_pt, d_seq, d_pos, d_k, d_v, conf, 0, 0.0625, split, n,
            len(seq)), "noalloc")
        torch.cuda.synchronize()

    call()
    free0 = torch.cuda.mem_get_info()[0]
    for _ in range(3):
        call()
    assert torch.cuda.mem_get_info()[0] == free0


def test_noalloc_rejects_calls_past_the_scratch(dev):
    import torch
    conf = gk.make_config(1, 64, 64, 1, 64, 8, 256, 0)
    dummy = torch.zeros(16, dtype=torch.int16, device=dev)
    i32 = torch.zeros(64, dtype=torch.int32, device=dev)
    # 64 sequences x 16 heads x 1024 splits x 258 floats is far past 40 MiB.
    code = gk.flash_attention_append_decode_paged_bf16_noalloc(
        dummy, dummy, dummy, dummy, i32, i32, i32, dummy, dummy, conf, 0, 0.0625, 64, 1024, 64)
    assert code == HIP_ERROR_OUT_OF_MEMORY
    # Counts past the entry point's limits are refused before the scratch
    # size is computed.
    for batch, splits in ((70000, 2), (1, 70000)):
        code = gk.flash_attention_append_decode_paged_bf16_noalloc(
            dummy, dummy, dummy, dummy, i32, i32, i32, dummy, dummy, conf, 0, 0.0625, 64,
            splits, batch)
        assert code == gk.HIP_ERROR_INVALID_VALUE
    torch.cuda.synchronize()
