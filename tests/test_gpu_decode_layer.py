"""One decode layer composed from the entry points, several steps in a row,
against the oracle chain (the reference layer order,
src/gemma4_flash_attention_decode.cu:979-1067 with the prep of :216-375 and
the output tail of :34-129):
  decode prep + append  (q/k/v RMSNorm + RoPE, the token's cache row)
  -> paged split-K decode attention over the cache, the new row included
  -> attention output projection + post-attention RMSNorm + residual.
Each step's metadata advances as the runtime's decode step does (position =
old length, length + 1), through a sliding ring that wraps. Bars: prepared
rows within one bf16 ulp of the oracle's (sum-of-squares order), attention
within the north-star tolerance of the oracle chain, the projection within
one ulp plus the fp32 summation bound of the oracle applied to the GPU's own
attention row, and within two ulps (plus a small absolute term for sums
that cancel) of the oracle chain end to end, after three bf16 roundings."""
import numpy as np
import pytest

import gemma_kv as gk
from kvtest import (assert_close, cache_config, empty_bf16, fill_page_table, from_dev_bf16,
                    randn_bf16, ring_pages, to_dev)
from oracle import oracle

pytestmark = pytest.mark.gpu

QH, HIDDEN = 16, 3840


def _ulp_diff(a_bits, b_bits):
    a = a_bits.astype(np.int32)
    b = b_bits.astype(np.int32)
    a = np.where(a & 0x8000, 0x8000 - (a & 0x7FFF), a + 0x8000)
    b = np.where(b & 0x8000, 0x8000 - (b & 0x7FFF), b + 0x8000)
    return np.abs(a - b)


def _close_chain(got_bits, exp_bits, what):
    """End of the chain: three bf16 roundings in sequence (attention row,
    residual, normed row), so two ulps of the value, plus an absolute term
    for sums that cancel (an attention-level ulp times the weights)."""
    got = oracle.bf16_to_f32(got_bits).astype(np.float64)
    exp = oracle.bf16_to_f32(exp_bits).astype(np.float64)
    err = np.abs(got - exp) - (np.abs(exp) * 2.0 ** -6 + 4e-3)
    assert err.max() <= 0, f"{what}: worst excess {err.max():.3g}"


def test_decode_layer_steps_against_oracle_chain(dev):
    import torch
    rng = np.random.default_rng(21)
    heads, dim, rotary, theta, window, page = 8, 256, 256, 10000.0, 64, 16
    seq0 = [70, 9]          # sequence 0 is past the window: its ring wraps during the steps
    steps = 4
    batch = len(seq0)
    max_pages = ring_pages(window, page)
    cfg_t = cache_config(1, batch, page, max_pages, heads, dim, window)
    cfg = gk.make_config(*cfg_t)
    rows = batch * max_pages * page
    ck_h = randn_bf16(rng, (rows, heads, dim))
    cv_h = randn_bf16(rng, (rows, heads, dim))
    qw = oracle.f32_to_bf16(1.0 + 0.2 * rng.standard_normal(dim).astype(np.float32))
    kw = oracle.f32_to_bf16(1.0 + 0.2 * rng.standard_normal(dim).astype(np.float32))
    post_w = oracle.f32_to_bf16(1.0 + 0.1 * rng.standard_normal(HIDDEN).astype(np.float32))
    w_o = randn_bf16(rng, (HIDDEN, QH * dim), scale=0.02)
    cos, sin = oracle.fill_rope_tables(256, rotary // 2, theta, dim)
    scale = 1.0 / 16.0
    half = rotary // 2

    d_ck, d_cv = to_dev(ck_h, dev), to_dev(cv_h, dev)
    d_w, d_post, d_qw, d_kw = to_dev(w_o, dev), to_dev(post_w, dev), to_dev(qw, dev), to_dev(kw, dev)
    d_cos, d_sin = to_dev(cos, dev), to_dev(sin, dev)
    split, n_splits = gk.decode_split_plan(cfg, batch, window)
    pm = torch.empty(batch * QH * n_splits, device=dev)
    pl = torch.empty_like(pm)
    pa = torch.empty(batch * QH * n_splits * dim, device=dev)
    seq = list(seq0)
    for step in range(steps):
        pos = list(seq)                   # the token of this step sits at the old length
        seq = [s + 1 for s in seq]
        print(f"decode layer step {step} positions {pos}", flush=True)
        pt = fill_page_table(cfg_t, seq)  # ring slots mapped up to the new length
        q = randn_bf16(rng, (batch, QH, dim))
        k = randn_bf16(rng, (batch, heads, dim), scale=2.0)
        v = randn_bf16(rng, (batch, heads, dim))
        x = randn_bf16(rng, (batch, HIDDEN))

        # ---- GPU chain
        d_pt = to_dev(pt, dev)
        d_pos = to_dev(np.asarray(pos, np.int32), dev)
        d_seq = to_dev(np.asarray(seq, np.int32), dev)
        d_qp = empty_bf16((batch, QH, dim), dev)
        gk.check(gk.decode_prep_append_bf16(d_qp, d_ck, d_cv, cfg, d_pt, d_pos, 0, to_dev(q, dev),
                                            to_dev(k, dev), to_dev(v, dev), d_qw, d_kw, d_cos,
                                            d_sin, batch), "decode prep")
        d_att = empty_bf16((batch, QH, dim), dev)
        gk.check(gk.flash_attention_decode_paged_bf16(d_att, pm, pl, pa, d_qp, d_ck, d_cv, d_pt,
                                                      d_seq, cfg, 0, scale, split, n_splits,
                                                      batch), "decode attention")
        outs = [empty_bf16((batch, HIDDEN), dev) for _ in range(3)]
        gk.check(gk.attention_o_projection_post_norm_bf16(
            *outs, d_att, d_w, d_post, to_dev(x, dev), batch, QH * dim), "o projection")
        torch.cuda.synchronize()
        got_qp = from_dev_bf16(d_qp).reshape(batch, QH, dim)
        got_att = from_dev_bf16(d_att).reshape(batch, QH, dim)
        got_res, got_norm, _ = (from_dev_bf16(t) for t in outs)

        # ---- oracle chain
        exp_qp = np.zeros((batch, QH, dim), np.uint16)
        kp = np.zeros((batch, heads, dim), np.uint16)
        vp = np.zeros((batch, heads, dim), np.uint16)
        for b, p in enumerate(pos):
            c_row, s_row = cos[p * half:(p + 1) * half], sin[p * half:(p + 1) * half]
            for h in range(QH):
                exp_qp[b, h] = oracle.prep_head(q[b, h], qw, c_row, s_row, rotary)
            for h in range(heads):
                kp[b, h] = oracle.prep_head(k[b, h], kw, c_row, s_row, rotary)
                vp[b, h] = oracle.prep_head(v[b, h], None, None, None, rotary)
        oracle.kv_cache_write(ck_h, cv_h, cfg_t, pt, np.arange(batch), pos, 0, kp, vp)
        exp_att = oracle.decode_attention(exp_qp, ck_h, cv_h, pt, seq, cfg_t, 0, scale)
        exp_res, exp_norm, _ = oracle.attention_o_projection(
            exp_att.reshape(batch, QH * dim), w_o, post_w, x)
        own_res, own_norm, _ = oracle.attention_o_projection(
            got_att.reshape(batch, QH * dim), w_o, post_w, x)

        d = _ulp_diff(got_qp, exp_qp)
        assert d.max() <= 1 and (d > 0).mean() < 0.02, ("q_prepared", step)
        assert_close(got_att, exp_att, f"attention step {step}")
        # Projection of the GPU's own attention row: one ulp plus the fp32 sum.
        a64 = np.abs(oracle.bf16_to_f32(got_att.reshape(batch, -1)).astype(np.float64))
        mag = a64 @ np.abs(oracle.bf16_to_f32(w_o).astype(np.float64)).T
        exp_own = oracle.bf16_to_f32(own_res).astype(np.float64)
        err = np.abs(oracle.bf16_to_f32(got_res) - exp_own)
        assert np.all(err <= np.abs(exp_own) * 2.0 ** -7 + 2.0 ** -16 * mag), ("residual", step)
        assert_close(got_norm, own_norm, f"normed step {step}")
        _close_chain(got_res, exp_res, f"residual vs chain step {step}")
        _close_chain(got_norm, exp_norm, f"normed vs chain step {step}")
    # The cache rows the GPU wrote equal the oracle's within one ulp; the rest
    # of the cache is untouched.
    got_k = from_dev_bf16(d_ck).reshape(ck_h.shape)
    got_v = from_dev_bf16(d_cv).reshape(cv_h.shape)
    assert _ulp_diff(got_k, ck_h).max() <= 1
    assert _ulp_diff(got_v, cv_h).max() <= 1


def test_prefill_then_decode_against_oracle(dev):
    """The prompt-then-decode handoff of one sliding layer: the prefill
    launcher (prep + causal windowed attention), the prefill cache write
    (only the last `window` rows of each sequence reach the ring,
    src/gemma4_prefill_megakernel.cu:189-207), then one decode step (prep +
    append + attention) over the cache the prefill left. The cache equals the
    oracle's write of the GPU's prepared rows bit for bit; attention outputs
    are within the north-star tolerance of the oracle."""
    import torch
    rng = np.random.default_rng(22)
    heads, dim, rotary, theta, window, page = 8, 256, 256, 10000.0, 64, 16
    batch, seq = 2, 100
    rows = batch * seq
    max_pages = ring_pages(window, page)
    cfg_t = cache_config(1, batch, page, max_pages, heads, dim, window)
    cfg = gk.make_config(*cfg_t)
    q = randn_bf16(rng, (rows, QH, dim))
    k = randn_bf16(rng, (rows, heads, dim), scale=2.0)
    v = randn_bf16(rng, (rows, heads, dim))
    qw = oracle.f32_to_bf16(1.0 + 0.2 * rng.standard_normal(dim).astype(np.float32))
    kw = oracle.f32_to_bf16(1.0 + 0.2 * rng.standard_normal(dim).astype(np.float32))
    cos, sin = oracle.fill_rope_tables(256, rotary // 2, theta, dim)
    pos = np.tile(np.arange(seq, dtype=np.int32), batch)
    tb = np.repeat(np.arange(batch, dtype=np.int32), seq)
    scale = 1.0 / 16.0
    half = rotary // 2
    d_cos, d_sin, d_qw, d_kw = to_dev(cos, dev), to_dev(sin, dev), to_dev(qw, dev), to_dev(kw, dev)

    print("prefill launcher", flush=True)
    out = empty_bf16((rows, QH, dim), dev)
    qp, kp, vp = (empty_bf16(s, dev) for s in ((rows, QH, dim), (rows, heads, dim),
                                                (rows, heads, dim)))
    gk.check(gk.flash_attention_sliding_fwd_bf16_norm_rope(
        out, qp, kp, vp, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), d_qw, d_kw, d_cos,
        d_sin, to_dev(pos, dev), batch, seq, seq, window, scale), "sliding launcher")
    pt = fill_page_table(cfg_t, [seq] * batch)
    d_pt = to_dev(pt, dev)
    cache_rows = batch * max_pages * page
    ck0 = randn_bf16(rng, (cache_rows, heads, dim))  # stale ring contents
    cv0 = randn_bf16(rng, (cache_rows, heads, dim))
    d_ck, d_cv = to_dev(ck0, dev), to_dev(cv0, dev)
    print("prefill cache write", flush=True)
    gk.check(gk.kv_cache_write_prefill_bf16(d_ck, d_cv, cfg, d_pt, to_dev(tb, dev),
                                            to_dev(pos, dev), batch, seq, 0, kp, vp),
             "prefill write")
    torch.cuda.synchronize()
    got_out = from_dev_bf16(out)
    kph = from_dev_bf16(kp).reshape(rows, heads, dim)
    vph = from_dev_bf16(vp).reshape(rows, heads, dim)
    qph = from_dev_bf16(qp).reshape(rows, QH, dim)
    # Prefill attention vs the oracle on the GPU's prepared rows.
    for b in range(batch):
        sl = slice(b * seq, (b + 1) * seq)
        exp = oracle.prefill_attention(qph[sl], kph[sl], vph[sl], seq, seq, QH, heads, dim,
                                       window, scale)
        assert_close(got_out.reshape(rows, QH, dim)[sl], exp, f"prefill attention batch {b}")
    # Cache: the oracle's write of the last `window` rows of each sequence.
    exp_ck, exp_cv = ck0.copy(), cv0.copy()
    tail = np.concatenate([np.arange(b * seq + seq - window, (b + 1) * seq) for b in range(batch)])
    oracle.kv_cache_write(exp_ck, exp_cv, cfg_t, pt, tb[tail], pos[tail], 0, kph[tail],
                          vph[tail])
    assert np.array_equal(from_dev_bf16(d_ck).reshape(exp_ck.shape), exp_ck)
    assert np.array_equal(from_dev_bf16(d_cv).reshape(exp_cv.shape), exp_cv)

    print("decode step after prefill", flush=True)
    dpos = [seq] * batch
    dseq = [seq + 1] * batch
    pt = fill_page_table(cfg_t, dseq)
    d_pt = to_dev(pt, dev)
    q1 = randn_bf16(rng, (batch, QH, dim))
    k1 = randn_bf16(rng, (batch, heads, dim), scale=2.0)
    v1 = randn_bf16(rng, (batch, heads, dim))
    d_qp1 = empty_bf16((batch, QH, dim), dev)
    gk.check(gk.decode_prep_append_bf16(d_qp1, d_ck, d_cv, cfg, d_pt,
                                        to_dev(np.asarray(dpos, np.int32), dev), 0,
                                        to_dev(q1, dev), to_dev(k1, dev), to_dev(v1, dev), d_qw,
                                        d_kw, d_cos, d_sin, batch), "decode prep")
    split, n_splits = gk.decode_split_plan(cfg, batch, window)
    pm = torch.empty(batch * QH * n_splits, device=dev)
    pl = torch.empty_like(pm)
    pa = torch.empty(batch * QH * n_splits * dim, device=dev)
    d_att = empty_bf16((batch, QH, dim), dev)
    gk.check(gk.flash_attention_decode_paged_bf16(d_att, pm, pl, pa, d_qp1, d_ck, d_cv, d_pt,
                                                  to_dev(np.asarray(dseq, np.int32), dev), cfg,
                                                  0, scale, split, n_splits, batch), "decode")
    torch.cuda.synchronize()
    exp_qp1 = np.zeros((batch, QH, dim), np.uint16)
    kp1 = np.zeros((batch, heads, dim), np.uint16)
    vp1 = np.zeros((batch, heads, dim), np.uint16)
    p = seq
    c_row, s_row = cos[p * half:(p + 1) * half], sin[p * half:(p + 1) * half]
    for b in range(batch):
        for h in range(QH):
            exp_qp1[b, h] = oracle.prep_head(q1[b, h], qw, c_row, s_row, rotary)
        for h in range(heads):
            kp1[b, h] = oracle.prep_head(k1[b, h], kw, c_row, s_row, rotary)
            vp1[b, h] = oracle.prep_head(v1[b, h], None, None, None, rotary)
    oracle.kv_cache_write(exp_ck, exp_cv, cfg_t, pt, np.arange(batch), dpos, 0, kp1, vp1)
    exp_att = oracle.decode_attention(exp_qp1, exp_ck, exp_cv, pt, dseq, cfg_t, 0, scale)
    assert_close(from_dev_bf16(d_att).reshape(batch, QH, dim), exp_att, "decode after prefill")
