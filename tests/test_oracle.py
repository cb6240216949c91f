"""Pins the CPU oracle before it is trusted as the checker.

Every check here is independent of the oracle's own formula: IEEE bit-level
known answers, the reference tests' known answers, brute-force enumeration,
a float64 library routine (torch's scaled_dot_product_attention on the CPU)
and closed forms chosen so that a dropped term, a wrong sign/index or a
transposed operand fails.
"""
import math

import numpy as np
import pytest

from kvtest import fill_page_table, make_prefill_value, make_value, randn_bf16, ring_pages
from oracle import oracle

torch = pytest.importorskip("torch")


# ---- bf16 conversion ---------------------------------------------------------

def test_bf16_round_to_nearest_even_known_answers():
    cases = [
        (1.0, 0x3F80), (-2.0, 0xC000), (0.0, 0x0000), (-0.0, 0x8000),
        (float.fromhex("0x1.01p0"), 0x3F80),    # exactly half an ulp above 1: ties to even (down)
        (float.fromhex("0x1.03p0"), 0x3F82),    # exactly half an ulp above odd 0x3F81: ties up
        (float.fromhex("0x1.0101p0"), 0x3F81),  # just above the tie: rounds up
        (float("inf"), 0x7F80), (-float("inf"), 0xFF80),
        (3.4e38, 0x7F80),                        # rounds up past the largest finite bf16
    ]
    for x, bits in cases:
        assert oracle.f32_to_bf16(np.float32(x)).item() == bits, x
    nan = oracle.f32_to_bf16(np.float32("nan")).item()
    assert (nan & 0x7F80) == 0x7F80 and (nan & 0x7F) != 0
    # Round trip of every bf16 pattern that is a number is the identity.
    allbits = np.arange(1 << 16, dtype=np.uint16)
    vals = oracle.bf16_to_f32(allbits)
    finite = ~np.isnan(vals)
    assert np.array_equal(oracle.f32_to_bf16(vals)[finite], allbits[finite])
    # Matches torch's bf16 rounding on random fp32 values.
    x = np.random.default_rng(0).standard_normal(100000).astype(np.float32) * 100
    ref = torch.from_numpy(x).bfloat16().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.f32_to_bf16(x), ref)


def test_make_value_generators_match_reference_formula_points():
    # tests/test_kv_cache.cu:42-45: seed 0 -> (17 % 257 - 128) / 64 = -1.734375
    assert oracle.bf16_to_f32(np.uint16(make_value(0))) == np.float32(-111 / 64)
    assert oracle.bf16_to_f32(np.uint16(make_value(3))) == np.float32((128 - 128) / 64)
    assert oracle.bf16_to_f32(np.uint16(make_prefill_value(0))) == np.float32(-117 / 512)


# ---- cache geometry / ring bookkeeping ----------------------------------------

def test_layout_offset_enumerates_every_slot_once():
    cfg = (2, 3, 4, 3, 1, 2, 8, 0)
    seen = []
    for layer in range(2):
        for page in range(3):
            for off in range(4):
                for head in range(2):
                    for dim in range(8):
                        seen.append(oracle.kv_cache_offset(cfg, layer, page, off, head, dim))
    assert seen == list(range(2 * 3 * 4 * 2 * 8))  # row-major [layer][page][off][head][dim]


def test_model_cadence_and_layer_index():
    glob = [l for l in range(48) if oracle.is_global_layer(l)]
    assert glob == [5, 11, 17, 23, 29, 35, 41, 47]
    assert [oracle.layer_index(l, True) for l in glob] == list(range(8))
    sliding = [l for l in range(48) if not oracle.is_global_layer(l)]
    assert [oracle.layer_index(l, False) for l in sliding] == list(range(40))
    assert oracle.layer_index(5, False) == -1 and oracle.layer_index(4, True) == -1
    assert oracle.layer_index(48, True) == -1 and oracle.layer_index(-1, False) == -1


def test_sliding_pages_per_sequence():
    # src/gemma4_runtime.cu:18-24: a window may straddle page boundaries.
    assert oracle.sliding_pages_per_sequence(1024, 1) == 1024
    assert oracle.sliding_pages_per_sequence(8192, 1) == 1024
    assert oracle.sliding_pages_per_sequence(8192, 64) == 17
    assert oracle.sliding_pages_per_sequence(66, 64) == 2
    assert oracle.sliding_pages_per_sequence(100000, 1000) == 3


def test_ensure_page_matches_reference_runtime_test():
    """tests/test_runtime_state.cu:29-107 (batch 2, max_seq 66, page 64):
    after prefill of 64 tokens and one decode step, slot 1 maps page 1 of each
    sequence; a position behind a newer page of the same slot is refused."""
    page, max_pages, batch = 64, 2, 2
    cfg = (1, batch * max_pages, page, max_pages, batch, 8, 256, 0)
    pt = np.full(batch * max_pages, -1, np.int32)
    slots = pt.copy()
    for b in range(batch):
        assert oracle.ensure_range(pt, slots, cfg, b, 0, 64) == 0
    assert pt[0] == 0 and pt[max_pages] == max_pages and pt[1] == -1
    for b in range(batch):
        assert oracle.ensure_page(pt, slots, cfg, b, 64) == b * max_pages + 1
    assert pt[1] == 1 and pt[max_pages + 1] == max_pages + 1
    # Ring reuse: a 2-slot ring, page 2 reuses slot 0; page 0 is then stale.
    assert oracle.ensure_page(pt, slots, cfg, 0, 128) == 0
    before = (pt.copy(), slots.copy())
    assert oracle.ensure_page(pt, slots, cfg, 0, 5) == -1
    assert np.array_equal(pt, before[0]) and np.array_equal(slots, before[1])


def test_invalid_row_write_known_answer():
    """tests/test_kv_cache.cu:94-133: a token whose batch row is out of range
    leaves the cache all zero."""
    cfg = (1, 2, 4, 2, 1, 2, 16, 0)
    ck = np.zeros(1 * 2 * 4 * 2 * 16, np.uint16)
    cv = np.zeros_like(ck)
    k = np.array([make_value(43000 + i) for i in range(32)], np.uint16)
    v = np.array([make_value(44000 + i) for i in range(32)], np.uint16)
    oracle.kv_cache_write(ck, cv, cfg, np.full(2, -1, np.int32), [1], [0], 0, k, v)
    assert not ck.any() and not cv.any()


def test_write_skip_rules_and_gather_round_trip():
    """Append semantics through invariants a wrong rule would fail, rather than
    a restatement of the rules (src/gemma4_kv_cache.cu:25-54):
    * a skipped row -- negative batch or position, batch past the config,
      unmapped slot, physical page out of range, a global position past
      max_pages_per_seq -- leaves a random cache byte-identical;
    * a written row is found again by the attention's own page-table gather
      (oracle_decode_attention over a window of one live key returns exactly
      that V row for any q), for global and for wrapped sliding positions;
    * a write changes exactly heads x head_dim elements of K and of V."""
    rng = np.random.default_rng(2)
    page, max_pages, batch, heads, dim, layers = 4, 3, 2, 2, 8, 2
    num_pages = batch * max_pages
    pt = np.array([0, 1, -1, 3, 9, 5], np.int32)  # b0 slot 2 unmapped, b1 slot 1 -> page 9 (out of range)
    size = layers * num_pages * page * heads * dim
    base_k = rng.integers(0, 1 << 16, size).astype(np.uint16)
    base_v = rng.integers(0, 1 << 16, size).astype(np.uint16)
    glob = (layers, num_pages, page, max_pages, batch, heads, dim, 0)
    slide = (layers, num_pages, page, max_pages, batch, heads, dim, 1)  # one live key

    def write(cfg, b, p):
        k = rng.integers(0, 1 << 15, (1, heads, dim)).astype(np.uint16)
        v = rng.integers(0, 1 << 15, (1, heads, dim)).astype(np.uint16)
        ck, cv = base_k.copy(), base_v.copy()
        oracle.kv_cache_write(ck, cv, cfg, pt, [b], [p], 1, k, v)
        return ck, cv, k, v

    skipped = [(glob, -1, 0), (glob, 0, -1), (glob, 2, 0), (glob, 0, 8), (glob, 0, 9),
               (glob, 1, 4), (glob, 0, 12), (glob, 1, 13), (slide, 0, 21), (slide, 1, 17)]
    for cfg, b, p in skipped:
        ck, cv, _, _ = write(cfg, b, p)
        assert np.array_equal(ck, base_k) and np.array_equal(cv, base_v), (cfg[7], b, p)

    written = [(glob, 0, 0), (glob, 0, 7), (glob, 1, 2), (glob, 1, 11),
               (slide, 0, 12), (slide, 0, 19), (slide, 1, 14), (slide, 1, 23)]
    for cfg, b, p in written:
        ck, cv, k, v = write(cfg, b, p)
        assert (ck != base_k).sum() <= heads * dim and (cv != base_v).sum() <= heads * dim
        assert (ck != base_k).sum() > heads * dim // 2  # random rows: almost all differ
        q = oracle.f32_to_bf16(rng.standard_normal((batch, 16, dim)).astype(np.float32))
        one = (layers, num_pages, page, max_pages, batch, heads, dim, 1)
        seq = np.zeros(batch, np.int32)
        seq[b] = p + 1
        out = oracle.decode_attention(q, ck, cv, pt, seq, one, 1, 0.125)
        group = 16 // heads
        for qh in range(16):
            assert np.array_equal(out[b, qh], v[0, qh // group]), (cfg[7], b, p, qh)


# ---- attention against a float64 library routine and closed forms --------------

def _sdpa64(q, k, v, mask, scale):
    """torch SDPA in float64 on the CPU. q [H, Lq, D], k/v [H, Lk, D], mask [Lq, Lk]."""
    tq = torch.from_numpy(q.astype(np.float64))
    tk = torch.from_numpy(k.astype(np.float64))
    tv = torch.from_numpy(v.astype(np.float64))
    tm = torch.from_numpy(mask)
    return torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, attn_mask=tm,
                                                            scale=scale).numpy()


@pytest.mark.parametrize("heads,dim,page,window,seq", [
    (8, 256, 1, 16, [37]), (8, 256, 4, 0, [21, 9]), (1, 512, 8, 0, [30]), (2, 16, 2, 6, [13, 4, 0]),
])
def test_decode_oracle_matches_float64_sdpa(heads, dim, page, window, seq):
    rng = np.random.default_rng(heads * 7 + dim)
    batch = len(seq)
    max_pages = ring_pages(window, page) if window else (max(max(seq), 1) + page - 1) // page
    cfg = (1, batch * max_pages, page, max_pages, batch, heads, dim, window)
    pt = fill_page_table(cfg, seq)
    rows = batch * max_pages * page
    ck = randn_bf16(rng, (rows, heads, dim))
    cv = randn_bf16(rng, (rows, heads, dim))
    q = randn_bf16(rng, (batch, 16, dim))
    scale = 1 / math.sqrt(dim)
    got = oracle.bf16_to_f32(oracle.decode_attention(q, ck, cv, pt, seq, cfg, 0, scale))
    kf, vf, qf = oracle.bf16_to_f32(ck), oracle.bf16_to_f32(cv), oracle.bf16_to_f32(q)
    group = 16 // heads
    for b, n in enumerate(seq):
        first = max(0, n - window) if window else 0
        keys = list(range(first, n))
        if not keys:
            assert not got[b].any()
            continue
        # Gather each key by walking the ring independently of the oracle.
        idx = [(pt[b * max_pages + (kk // page) % max_pages]) * page + kk % page for kk in keys]
        kk_ = kf[idx].transpose(1, 0, 2)  # [heads, n, dim]
        vv_ = vf[idx].transpose(1, 0, 2)
        for qh in range(16):
            ref = _sdpa64(qf[b, qh][None, None], kk_[qh // group][None], vv_[qh // group][None],
                          np.ones((1, len(keys)), bool), scale)[0, 0]
            np.testing.assert_allclose(got[b, qh], ref, atol=1e-2, rtol=1e-2)


def test_decode_oracle_closed_forms():
    rng = np.random.default_rng(9)
    heads, dim, page, window = 8, 256, 1, 64
    cfg = (1, 64, page, 64, 1, heads, dim, window)
    seq = [200]
    pt = fill_page_table(cfg, seq)
    ck = randn_bf16(rng, (64, heads, dim))
    cv = randn_bf16(rng, (64, heads, dim))
    # q = 0: uniform weights -> mean of the 64 live V rows per kv head.
    out = oracle.bf16_to_f32(oracle.decode_attention(np.zeros((1, 16, dim), np.uint16), ck, cv,
                                                     pt, seq, cfg, 0, 0.0625))
    mean = oracle.bf16_to_f32(cv).astype(np.float64).mean(axis=0)
    assert np.abs(out[0] - np.repeat(mean, 2, axis=0)).max() < 4e-3
    # One live key -> that key's V row, exactly (weight 1).
    pt1 = fill_page_table(cfg, [1])
    out1 = oracle.decode_attention(randn_bf16(rng, (1, 16, dim)), ck, cv, pt1, [1], cfg, 0, 0.0625)
    assert np.array_equal(out1[0].reshape(8, 2, dim)[:, 0], cv[0])
    # Window: keys older than seq - window have no effect at all.
    q = randn_bf16(rng, (1, 16, dim))
    cfg_big = (1, 256, 1, 256, 1, heads, dim, window)
    ptb = fill_page_table(cfg_big, [200])
    bk = randn_bf16(rng, (256, heads, dim))
    bv = randn_bf16(rng, (256, heads, dim))
    a = oracle.decode_attention(q, bk, bv, ptb, [200], cfg_big, 0, 0.0625)
    bk2, bv2 = bk.copy(), bv.copy()
    bk2[:136] = randn_bf16(rng, (136, heads, dim))
    bv2[:136] = randn_bf16(rng, (136, heads, dim))
    assert np.array_equal(a, oracle.decode_attention(q, bk2, bv2, ptb, [200], cfg_big, 0, 0.0625))
    # Key permutation invariance through the page table (page 1 -> any slot order).
    perm = rng.permutation(256).astype(np.int32)
    pk = np.empty_like(bk)
    pv = np.empty_like(bv)
    pk[perm] = bk
    pv[perm] = bv
    out_p = oracle.decode_attention(q, pk, pv, perm, [200], cfg_big, 0, 0.0625)
    assert np.abs(oracle.bf16_to_f32(out_p) - oracle.bf16_to_f32(a)).max() <= 2 ** -7


def test_split_partials_and_combine_equal_unsplit():
    rng = np.random.default_rng(4)
    heads, dim, page = 8, 256, 16
    seq = [333, 1]
    cfg = (1, 2 * 32, page, 32, 2, heads, dim, 0)
    pt = fill_page_table(cfg, seq)
    ck = randn_bf16(rng, (2 * 32 * page, heads, dim), scale=2.0)
    cv = randn_bf16(rng, (2 * 32 * page, heads, dim))
    q = randn_bf16(rng, (2, 16, dim))
    direct = oracle.bf16_to_f32(oracle.decode_attention(q, ck, cv, pt, seq, cfg, 0, 0.0625))
    for split in (1, 7, 50, 333, 512):
        n = (max(seq) + split - 1) // split
        pm, pl, pa = oracle.decode_split(q, ck, cv, pt, seq, cfg, 0, 0.0625, split, n)
        comb = oracle.bf16_to_f32(oracle.decode_combine(pm, pl, pa, seq, cfg, split, n))
        assert np.abs(comb - direct).max() <= 2 ** -6, split
        # The sequence with one key has exactly one live split per row.
        assert np.isnan(pm.reshape(2, 16, n)[1, :, 1:]).all()


@pytest.mark.parametrize("window,lq,lk", [(0, 33, 33), (0, 17, 40), (8, 20, 20), (8, 12, 30), (5, 9, 4)])
def test_prefill_oracle_matches_float64_sdpa(window, lq, lk):
    rng = np.random.default_rng(lq * 100 + lk)
    heads, dim = 2, 32
    q = randn_bf16(rng, (1, lq, 16, dim))
    k = randn_bf16(rng, (1, lk, heads, dim))
    v = randn_bf16(rng, (1, lk, heads, dim))
    got = oracle.bf16_to_f32(oracle.prefill_attention(q, k, v, lq, lk, 16, heads, dim, window, 0.25))
    qf, kf, vf = (oracle.bf16_to_f32(x) for x in (q, k, v))
    mask = np.zeros((lq, lk), bool)
    for r in range(lq):
        kr = r + lk - lq
        lo = max(0, kr - window + 1) if window else 0
        mask[r, lo:max(0, min(lk, kr + 1))] = True
    for qh in range(16):
        kv = qh // (16 // heads)
        ok = mask.any(axis=1)
        ref = _sdpa64(qf[0, :, qh][None], kf[0, :, kv][None], vf[0, :, kv][None],
                      np.where(ok[:, None], mask, True), 0.25)[0]
        np.testing.assert_allclose(got[0, ok, qh], ref[ok], atol=1e-2, rtol=1e-2)
        assert not got[0, ~ok, qh].any()  # no visible key -> zeros


def test_prefill_q_zero_running_mean_known_answer():
    """tests/test_flash_attention.cu:335-345: with q = 0, causal row r is the
    mean of V rows 0..r."""
    lq, heads, dim = 6, 1, 512
    v = np.array([make_value(110000 + i) for i in range(lq * dim)], np.uint16).reshape(1, lq, 1, dim)
    k = np.array([make_value(7 + i) for i in range(lq * dim)], np.uint16).reshape(1, lq, 1, dim)
    q = np.zeros((1, lq, 16, dim), np.uint16)
    got = oracle.bf16_to_f32(oracle.prefill_attention(q, k, v, lq, lq, 16, heads, dim, 0, 1 / math.sqrt(dim)))
    vf = oracle.bf16_to_f32(v)[0, :, 0].astype(np.float64)
    for r in range(lq):
        exp = vf[:r + 1].mean(axis=0)
        assert np.abs(got[0, r] - exp[None]).max() <= 0.03125


# ---- Q/K preparation helpers ----------------------------------------------------

def test_rope_tables_match_reference_runtime_test():
    """tests/test_runtime_state.cu:110-140: sliding cos/sin at position 1,
    pair 0 is cos(1)/sin(1); global p-RoPE pair 1 at position 1 uses
    theta^(-2/512)."""
    cs, sn = oracle.fill_rope_tables(4, 128, 10000.0, 256)
    assert abs(cs[128] - math.cos(1.0)) < 1e-6 and abs(sn[128] - math.sin(1.0)) < 1e-6
    gc, _ = oracle.fill_rope_tables(4, 64, 1_000_000.0, 512)
    assert abs(gc[64 + 1] - math.cos(1_000_000.0 ** (-2.0 / 512))) < 1e-6


def test_prep_head_known_answers():
    """tests/test_flash_attention.cu:285-333: K-derived V is the scale-free
    RMSNorm of K; RoPE with (cos, sin) = (0, +-1) swaps the pair with a sign."""
    dim, half = 512, 64
    k = np.array([make_value(110000 + i) for i in range(dim)], np.uint16)
    kf = oracle.bf16_to_f32(k).astype(np.float64)
    inv = 1.0 / math.sqrt((kf ** 2).sum() / dim + 1e-6)
    v = oracle.bf16_to_f32(oracle.prep_head(k, None, None, None, 128))
    assert np.abs(v - kf * inv).max() <= 2 ** -8
    ones = np.full(dim, 0x3F80, np.uint16)
    cos = np.ones(half, np.float32)
    sin = np.zeros(half, np.float32)
    cos[0], sin[0] = 0.0, 1.0
    out = oracle.bf16_to_f32(oracle.prep_head(k, ones, cos, sin, 128))
    lo, hi = kf[0] * inv, kf[half] * inv
    assert abs(out[0] - (-hi)) <= 2 ** -7 and abs(out[half] - lo) <= 2 ** -7
    assert np.abs(out[1:half] - kf[1:half] * inv).max() <= 2 ** -7   # cos 1, sin 0: identity
    assert np.abs(out[128:] - kf[128:] * inv).max() <= 2 ** -7       # non-rotary tail


# ---- attention output projection + post-attention norm -----------------------

def _bf16_round(x):
    return oracle.f32_to_bf16(np.asarray(x, dtype=np.float32))


def test_o_projection_oracle_matches_float64_matmul():
    rng = np.random.default_rng(7)
    rows, width, hidden = 3, 512, 384
    attn = randn_bf16(rng, (rows, width))
    w = _bf16_round(rng.standard_normal((hidden, width)) * 0.05)
    g = _bf16_round(1.0 + 0.1 * rng.standard_normal(hidden))
    x = randn_bf16(rng, (rows, hidden))
    res, normed, ffn = oracle.attention_o_projection(attn, w, g, x)
    a64 = oracle.bf16_to_f32(attn).astype(np.float64)
    w64 = oracle.bf16_to_f32(w).astype(np.float64)
    want = _bf16_round(a64 @ w64.T)
    diff = np.abs(res.astype(np.int32) - want.astype(np.int32))
    assert diff.max() <= 1 and (diff == 0).mean() > 0.999
    # RMSNorm of the bf16 residual row with the learned weight, in float64.
    r64 = oracle.bf16_to_f32(res).astype(np.float64)
    scale = 1.0 / np.sqrt((r64 ** 2).mean(axis=1, keepdims=True) + 1e-6)
    n64 = r64 * scale * oracle.bf16_to_f32(g).astype(np.float64)
    got = oracle.bf16_to_f32(normed).astype(np.float64)
    assert np.all(np.abs(got - n64) <= np.abs(n64) * 2.0 ** -8 + 1e-30)
    # Residual: x + normed, one rounding.
    s64 = oracle.bf16_to_f32(x).astype(np.float64) + got
    assert np.array_equal(ffn, _bf16_round(s64))


def test_o_projection_oracle_closed_forms():
    rng = np.random.default_rng(8)
    width, hidden = 256, 128
    w = _bf16_round(rng.standard_normal((hidden, width)))
    g = _bf16_round(0.5 + rng.random(hidden))
    # A one-hot attention row selects one weight element per hidden column
    # (catches a transposed weight: a column-major read would pick W[e0][c]).
    e0 = 37
    attn = np.zeros((1, width), dtype=np.uint16)
    attn[0, e0] = 0x3F80  # 1.0
    x = np.zeros((1, hidden), dtype=np.uint16)
    res, normed, ffn = oracle.attention_o_projection(attn, w, g, x)
    assert np.array_equal(res[0], w[:, e0])
    assert np.array_equal(ffn, normed)  # x = 0
    # A constant residual row (every W[c][e0] = 2) normalises to the weight.
    w2 = w.copy()
    w2[:, e0] = 0x4000  # 2.0
    res, normed, _ = oracle.attention_o_projection(attn, w2, g, x)
    assert np.all(res == 0x4000)
    assert np.abs(normed.astype(np.int32) - g.astype(np.int32)).max() <= 1
    # Negating the attention row negates the residual and the normed row.
    attn_neg = attn ^ np.uint16(0x8000)
    r1, n1, _ = oracle.attention_o_projection(attn, w, g, x)
    r2, n2, _ = oracle.attention_o_projection(attn_neg, w, g, x)
    assert np.array_equal(r1 ^ np.uint16(0x8000), r2)
    assert np.array_equal(n1 ^ np.uint16(0x8000), n2)
