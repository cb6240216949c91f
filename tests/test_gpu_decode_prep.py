"""Parity of the decode-token preparation + cache append
(gemma4_decode_prep_append_bf16, the reference's
phase_decode_q_paged_kv_norm_rope) against the oracle's prep_head applied per
head: learned RMSNorm + split-half RoPE for q and k, scale-free RMSNorm for v
(K-derived for the global geometry), written into the ring slot of the
token. The sum of squares is reduced in a different order on the GPU, so a
prepared value may differ from the oracle's by one bf16 ulp; anything larger
fails. Skip rules (negative position, unmapped page) are exact."""
import numpy as np
import pytest

import gemma_kv as gk
from kvtest import cache_config, fill_page_table, from_dev_bf16, randn_bf16, ring_pages, to_dev
from oracle import oracle

pytestmark = pytest.mark.gpu


def _ulp_diff(a_bits, b_bits):
    a = a_bits.astype(np.int32)
    b = b_bits.astype(np.int32)
    # bf16 bit patterns as sign-magnitude -> monotonic integers
    a = np.where(a & 0x8000, 0x8000 - (a & 0x7FFF), a + 0x8000)
    b = np.where(b & 0x8000, 0x8000 - (b & 0x7FFF), b + 0x8000)
    return np.abs(a - b)


def _close_bits(got, exp, what):
    d = _ulp_diff(got, exp)
    assert d.max(initial=0) <= 1, f"{what}: max ulp diff {d.max()}"
    assert (d > 0).mean() < 0.02, f"{what}: {(d > 0).mean():.3%} values differ"


@pytest.mark.parametrize("geometry", ["sliding", "global"])
def test_prep_append_against_oracle(dev, geometry):
    import torch
    rng = np.random.default_rng(11 if geometry == "sliding" else 12)
    if geometry == "sliding":
        heads, dim, rotary, theta, window, page = 8, 256, 256, 10000.0, 64, 1
    else:
        heads, dim, rotary, theta, window, page = 1, 512, 128, 1_000_000.0, 0, 16
    seq = [151, 9, 40]
    pos = [150, -1, 39]             # sequence 1 has no token this step
    batch = len(seq)
    max_pages = ring_pages(window, page) if window else (max(seq) + page - 1) // page
    layers = 2
    cfg = cache_config(layers, batch, page, max_pages, heads, dim, window)
    pt = fill_page_table(cfg, seq)
    # Unmap sequence 2's page of its token: q is still prepared, K/V skipped.
    lp = pos[2] // page
    pt[2 * max_pages + lp % max_pages] = -1
    rows = layers * batch * max_pages * page
    ck0 = randn_bf16(rng, (rows, heads, dim))
    cv0 = randn_bf16(rng, (rows, heads, dim))
    q = randn_bf16(rng, (batch, 16, dim))
    k = randn_bf16(rng, (batch, heads, dim), scale=3.0)
    v = randn_bf16(rng, (batch, heads, dim))
    qw = oracle.f32_to_bf16(1.0 + 0.2 * rng.standard_normal(dim).astype(np.float32))
    kw = oracle.f32_to_bf16(1.0 + 0.2 * rng.standard_normal(dim).astype(np.float32))
    cos, sin = oracle.fill_rope_tables(256, rotary // 2, theta, dim)
    layer = 1

    exp_q = np.full((batch, 16, dim), 0x7FC1, np.uint16)
    exp_k, exp_v = ck0.copy(), cv0.copy()
    half = rotary // 2
    for b, p in enumerate(pos):
        if p < 0:
            continue
        c_row, s_row = cos[p * half:(p + 1) * half], sin[p * half:(p + 1) * half]
        for h in range(16):
            exp_q[b, h] = oracle.prep_head(q[b, h], qw, c_row, s_row, rotary)
        phys = pt[b * max_pages + (p // page) % max_pages]
        if phys < 0:
            continue
        row = (layer * batch * max_pages + phys) * page + p % page
        for h in range(heads):
            exp_k[row, h] = oracle.prep_head(k[b, h], kw, c_row, s_row, rotary)
            exp_v[row, h] = oracle.prep_head(v[b, h] if geometry == "sliding" else k[b, h],
                                             None, None, None, rotary)

    ck, cv = to_dev(ck0, dev), to_dev(cv0, dev)
    qp = to_dev(np.full((batch, 16, dim), 0x7FC1, np.uint16), dev)
    code = gk.decode_prep_append_bf16(
        qp, ck, cv, gk.make_config(*cfg), to_dev(pt, dev), to_dev(np.asarray(pos, np.int32), dev),
        layer, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev) if geometry == "sliding" else None,
        to_dev(qw, dev), to_dev(kw, dev), to_dev(cos, dev), to_dev(sin, dev), batch)
    gk.check(code, "decode_prep_append")
    torch.cuda.synchronize()
    got_q = from_dev_bf16(qp).reshape(exp_q.shape)
    assert np.array_equal(got_q[1], exp_q[1])       # position -1: untouched
    _close_bits(got_q[[0, 2]], exp_q[[0, 2]], "q_prepared")
    got_k = from_dev_bf16(ck).reshape(exp_k.shape)
    got_v = from_dev_bf16(cv).reshape(exp_v.shape)
    changed = np.any(exp_k != ck0, axis=(1, 2)) | np.any(exp_v != cv0, axis=(1, 2))
    assert changed.sum() == 1                        # only sequence 0's row
    assert np.array_equal(got_k[~changed], ck0[~changed])
    assert np.array_equal(got_v[~changed], cv0[~changed])
    _close_bits(got_k[changed], exp_k[changed], "cache K")
    _close_bits(got_v[changed], exp_v[changed], "cache V")


def test_prep_append_argument_checks(dev):
    import torch
    cfg = gk.make_config(*cache_config(1, 1, 1, 64, 8, 128, 64))  # unsupported geometry
    z = torch.zeros(16, dtype=torch.int32, device=dev)
    assert gk.decode_prep_append_bf16(z, z, z, cfg, z, z, 0, z, z, z, z, z, z, z, 1) != 0
    cfg = gk.make_config(*cache_config(1, 1, 1, 64, 8, 256, 64))
    assert gk.decode_prep_append_bf16(z, z, z, cfg, z, z, 0, z, z, z, z, z, z, z, 0) == 0
    assert gk.decode_prep_append_bf16(z, z, z, cfg, z, z, 1, z, z, z, z, z, z, z, 1) != 0
    torch.cuda.synchronize()


@pytest.mark.parametrize("geometry,counters", [("sliding", False), ("sliding", True),
                                               ("global", False)])
def test_fused_prep_append_decode(dev, geometry, counters):
    """gemma4_flash_attention_prep_append_decode_paged_bf16 (one launch)
    against the oracle: the appended cache rows within one bf16 ulp of
    oracle.prep_head, everything else in the cache untouched, the attention
    outputs within the north-star tolerance of the oracle's attention over
    the oracle-prepared rows. A sequence with no token this step
    (position -1) appends nothing and attends with its q as given."""
    import torch
    from kvtest import assert_close
    rng = np.random.default_rng(31 if geometry == "sliding" else 32)
    if geometry == "sliding":
        heads, dim, rotary, theta, window, page = 8, 256, 256, 10000.0, 64, 16
    else:
        heads, dim, rotary, theta, window, page = 1, 512, 128, 1_000_000.0, 0, 16
    seq = [151, 40, 9]
    pos = [150, 39, -1]
    batch = len(seq)
    max_pages = ring_pages(window, page) if window else (max(seq) + page - 1) // page
    layers = 2
    cfg_t = cache_config(layers, batch, page, max_pages, heads, dim, window)
    pt = fill_page_table(cfg_t, seq)
    rows = layers * batch * max_pages * page
    ck0 = randn_bf16(rng, (rows, heads, dim))
    cv0 = randn_bf16(rng, (rows, heads, dim))
    q = randn_bf16(rng, (batch, 16, dim))
    k = randn_bf16(rng, (batch, heads, dim), scale=3.0)
    v = randn_bf16(rng, (batch, heads, dim))
    qw = oracle.f32_to_bf16(1.0 + 0.2 * rng.standard_normal(dim).astype(np.float32))
    kw = oracle.f32_to_bf16(1.0 + 0.2 * rng.standard_normal(dim).astype(np.float32))
    cos, sin = oracle.fill_rope_tables(256, rotary // 2, theta, dim)
    layer = 1
    scale = 1.0 / np.sqrt(dim)
    half = rotary // 2
    exp_k, exp_v = ck0.copy(), cv0.copy()
    q_used = q.copy()
    for b, p in enumerate(pos):
        if p < 0:
            continue
        c_row, s_row = cos[p * half:(p + 1) * half], sin[p * half:(p + 1) * half]
        for h in range(16):
            q_used[b, h] = oracle.prep_head(q[b, h], qw, c_row, s_row, rotary)
        row = (layer * batch * max_pages + pt[b * max_pages + (p // page) % max_pages]) * page + p % page
        for h in range(heads):
            exp_k[row, h] = oracle.prep_head(k[b, h], kw, c_row, s_row, rotary)
            exp_v[row, h] = oracle.prep_head(v[b, h] if geometry == "sliding" else k[b, h],
                                             None, None, None, rotary)
    exp_out = oracle.decode_attention(q_used, exp_k, exp_v, pt, seq, cfg_t, layer, scale)

    cfg = gk.make_config(*cfg_t)
    split, n = gk.decode_split_plan(cfg, batch, max(seq))
    pm = torch.empty(batch * 16 * n, device=dev)
    pl = torch.empty_like(pm)
    pa = torch.empty(batch * 16 * n * dim, device=dev)
    cnt = torch.zeros(batch * heads, dtype=torch.int32, device=dev) if counters else None
    ck, cv = to_dev(ck0, dev), to_dev(cv0, dev)
    out = torch.zeros((batch, 16, dim), dtype=torch.int16, device=dev)
    print(f"fused prep+decode {geometry} counters={counters} split {split}x{n}", flush=True)
    gk.check(gk.flash_attention_prep_append_decode_paged_bf16(
        out, pm, pl, pa, to_dev(q, dev), ck, cv, to_dev(pt, dev),
        to_dev(np.asarray(seq, np.int32), dev), to_dev(np.asarray(pos, np.int32), dev),
        to_dev(k, dev), to_dev(v, dev) if geometry == "sliding" else None, to_dev(qw, dev),
        to_dev(kw, dev), to_dev(cos, dev), to_dev(sin, dev), cfg, layer, scale, split, n, batch,
        split_counters=cnt), "fused prep+decode")
    torch.cuda.synchronize()
    got_k = from_dev_bf16(ck).reshape(exp_k.shape)
    got_v = from_dev_bf16(cv).reshape(exp_v.shape)
    changed = np.any(exp_k != ck0, axis=(1, 2)) | np.any(exp_v != cv0, axis=(1, 2))
    assert changed.sum() == 2
    assert np.array_equal(got_k[~changed], ck0[~changed])
    assert np.array_equal(got_v[~changed], cv0[~changed])
    _close_bits(got_k[changed], exp_k[changed], "cache K")
    _close_bits(got_v[changed], exp_v[changed], "cache V")
    assert_close(from_dev_bf16(out).reshape(exp_out.shape), exp_out, "attention")
    if counters:
        assert int(cnt.abs().sum().item()) == 0


def test_fused_prep_append_decode_argument_checks(dev):
    import torch
    cfg = gk.make_config(*cache_config(1, 1, 1, 64, 8, 256, 64))
    z = torch.zeros(64, dtype=torch.int32, device=dev)
    f = gk.flash_attention_prep_append_decode_paged_bf16
    # 8x256 needs v; weights and tables are required.
    assert f(z, z, z, z, z, z, z, z, z, z, z, None, z, z, z, z, cfg, 0, 0.0625, 32, 2, 1) != 0
    assert f(z, z, z, z, z, z, z, z, z, z, z, z, None, z, z, z, cfg, 0, 0.0625, 32, 2, 1) != 0
    assert f(z, z, z, z, z, z, z, z, z, None, z, z, z, z, z, z, cfg, 0, 0.0625, 32, 2, 1) != 0
    torch.cuda.synchronize()
