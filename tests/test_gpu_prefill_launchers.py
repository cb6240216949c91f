"""Prefill self-attention launchers with Q/K/V preparation
(gemma4_flash_attention_{sliding,global}_fwd_bf16_norm_rope): the reference's
own known-answer cases (tests/test_flash_attention.cu:175-346: global D512
seq 33 against a CPU reference at tolerance 1/32, and the K-derived V,
absolute-position RoPE and q = 0 running-mean case), then seeded random cases
on both geometries against the oracle: prepared rows within one bf16 ulp of
oracle.prep_head (the GPU sums squares in another order), attention outputs
against oracle.prefill_attention on the prepared rows within the north-star
tolerance."""
import math

import numpy as np
import pytest

import gemma_kv as gk
from kvtest import assert_close, empty_bf16, from_dev_bf16, make_prefill_value, make_value, randn_bf16, to_dev
from oracle import oracle

pytestmark = pytest.mark.gpu

QH = 16


def _ulp_diff(a_bits, b_bits):
    a = a_bits.astype(np.int32)
    b = b_bits.astype(np.int32)
    a = np.where(a & 0x8000, 0x8000 - (a & 0x7FFF), a + 0x8000)
    b = np.where(b & 0x8000, 0x8000 - (b & 0x7FFF), b + 0x8000)
    return np.abs(a - b)


def _close_bits(got, exp, what):
    d = _ulp_diff(got, exp)
    assert d.max(initial=0) <= 1, f"{what}: max ulp diff {d.max()}"
    assert (d > 0).mean() < 0.02, f"{what}: {(d > 0).mean():.3%} values differ"


def _run_global(dev, q, k, qw, kw, cos, sin, pos, batch, seq, scale):
    import torch
    rows = batch * seq
    out = empty_bf16((rows, QH, 512), dev)
    qp, kp, vp = empty_bf16((rows, QH, 512), dev), empty_bf16((rows, 1, 512), dev), empty_bf16((rows, 1, 512), dev)
    gk.check(gk.flash_attention_global_fwd_bf16_norm_rope(
        out, qp, kp, vp, to_dev(q, dev), to_dev(k, dev), to_dev(qw, dev), to_dev(kw, dev),
        to_dev(cos, dev), to_dev(sin, dev), to_dev(np.asarray(pos, np.int32), dev), batch, seq,
        seq, scale), "global launcher")
    torch.cuda.synchronize()
    return [from_dev_bf16(t) for t in (out, qp, kp, vp)]


def test_global_d512_seq33_reference_case(dev):
    """tests/test_flash_attention.cu:175-229: make_prefill_value inputs, unit
    norm weights, identity RoPE tables, positions 0..32; out against the CPU
    attention of the device-prepared rows at 1/32 (the reference's bar) and at
    the north-star tolerance."""
    seq, rot_half = 33, 512 // 8
    q = np.array([make_prefill_value(4000 + i) for i in range(seq * QH * 512)], np.uint16).reshape(seq, QH, 512)
    k = np.array([make_prefill_value(5000 + i) for i in range(seq * 512)], np.uint16).reshape(seq, 1, 512)
    w = np.full(512, oracle.f32_to_bf16(np.float32(1.0)), np.uint16)
    cos = np.ones(seq * rot_half, np.float32)
    sin = np.zeros(seq * rot_half, np.float32)
    scale = 1 / math.sqrt(512)
    out, qp, kp, vp = _run_global(dev, q, k, w, w, cos, sin, np.arange(seq), 1, seq, scale)
    exp = oracle.prefill_attention(qp.reshape(1, seq, QH, 512), kp.reshape(1, seq, 1, 512),
                                   vp.reshape(1, seq, 1, 512), seq, seq, QH, 1, 512, 0, scale)
    got = oracle.bf16_to_f32(out).reshape(exp.shape)
    assert np.abs(got - oracle.bf16_to_f32(exp)).max() <= 0.03125
    assert_close(out.reshape(exp.shape), exp, "global D512 seq 33")
    # The prepared rows themselves against the oracle's prep.
    exp_q = np.stack([oracle.prep_head(q[r, h], w, cos[:rot_half], sin[:rot_half], 128)
                      for r in range(seq) for h in range(QH)]).reshape(seq, QH, 512)
    _close_bits(qp.reshape(exp_q.shape), exp_q, "q_prepared")


def test_global_k_derived_v_and_absolute_rope(dev):
    """tests/test_flash_attention.cu:231-346: seq 2 at positions {2, 4} with
    cos/sin rotating pair 0 by +-90 degrees, q = 0: V is the scale-free norm
    of the raw K, K's pair 0 is rotated at the absolute position, and the
    outputs are v0 and the mean of v0 and v1 (1/256 and 1/32 tolerances)."""
    seq, rot_half = 2, 512 // 8
    k = np.array([make_value(110000 + i) for i in range(seq * 512)], np.uint16).reshape(seq, 1, 512)
    w = np.full(512, oracle.f32_to_bf16(np.float32(1.0)), np.uint16)
    pos = [2, 4]
    cos = np.ones(5 * rot_half, np.float32)
    sin = np.zeros(5 * rot_half, np.float32)
    cos[2 * rot_half], sin[2 * rot_half] = 0.0, 1.0
    cos[4 * rot_half], sin[4 * rot_half] = 0.0, -1.0
    q = np.zeros((seq, QH, 512), np.uint16)
    out, qp, kp, vp = _run_global(dev, q, k, w, w, cos, sin, pos, 1, seq, 1 / math.sqrt(512))
    kf = oracle.bf16_to_f32(k.reshape(seq, 512))
    inv_rms = 1.0 / np.sqrt((kf.astype(np.float32) ** 2).sum(1) / 512 + 1e-6)
    exp_v = oracle.bf16_to_f32(oracle.f32_to_bf16((kf * inv_rms[:, None]).astype(np.float32)))
    assert np.abs(oracle.bf16_to_f32(vp).reshape(seq, 512) - exp_v).max() <= 1 / 256
    kpf = oracle.bf16_to_f32(kp).reshape(seq, 512)
    for r in range(seq):
        c, s = cos[pos[r] * rot_half], sin[pos[r] * rot_half]
        lo, hi = kf[r, 0] * inv_rms[r], kf[r, rot_half] * inv_rms[r]
        e_lo = oracle.bf16_to_f32(oracle.f32_to_bf16(np.float32(lo * c - hi * s)))
        e_hi = oracle.bf16_to_f32(oracle.f32_to_bf16(np.float32(lo * s + hi * c)))
        assert abs(kpf[r, 0] - e_lo) <= 1 / 256 and abs(kpf[r, rot_half] - e_hi) <= 1 / 256, r
    vpf = oracle.bf16_to_f32(vp).reshape(seq, 512)
    got = oracle.bf16_to_f32(out).reshape(seq, QH, 512)
    assert np.abs(got[0] - vpf[0][None, :]).max() <= 0.03125
    assert np.abs(got[1] - (0.5 * (vpf[0] + vpf[1]))[None, :]).max() <= 0.03125


@pytest.mark.parametrize("batch,seq", [(1, 77), (2, 130)])
def test_global_random_against_oracle(dev, batch, seq):
    rng = np.random.default_rng(seq)
    rows = batch * seq
    q = randn_bf16(rng, (rows, QH, 512))
    k = randn_bf16(rng, (rows, 1, 512))
    qw = oracle.f32_to_bf16(1.0 + 0.2 * rng.standard_normal(512).astype(np.float32))
    kw = oracle.f32_to_bf16(1.0 + 0.2 * rng.standard_normal(512).astype(np.float32))
    cos, sin = oracle.fill_rope_tables(256, 64, 1_000_000.0, 512)
    pos = np.tile(np.arange(seq) + 3, batch)
    scale = 1 / math.sqrt(512)
    out, qp, kp, vp = _run_global(dev, q, k, qw, kw, cos, sin, pos, batch, seq, scale)
    r = rows - 1
    c_row, s_row = cos[pos[r] * 64:(pos[r] + 1) * 64], sin[pos[r] * 64:(pos[r] + 1) * 64]
    _close_bits(kp.reshape(rows, 512)[r], oracle.prep_head(k[r, 0], kw, c_row, s_row, 128), "k_prepared")
    _close_bits(vp.reshape(rows, 512)[r], oracle.prep_head(k[r, 0], None, None, None, 128), "v_prepared")
    exp = oracle.prefill_attention(qp.reshape(batch, seq, QH, 512), kp.reshape(batch, seq, 1, 512),
                                   vp.reshape(batch, seq, 1, 512), seq, seq, QH, 1, 512, 0, scale,
                                   batch=batch)
    assert_close(out.reshape(exp.shape), exp, f"global batch={batch} seq={seq}")


@pytest.mark.parametrize("batch,seq,window", [(1, 100, 32), (2, 70, 1024)])
def test_sliding_random_against_oracle(dev, batch, seq, window):
    import torch
    rng = np.random.default_rng(seq + window)
    rows = batch * seq
    q = randn_bf16(rng, (rows, QH, 256))
    k = randn_bf16(rng, (rows, 8, 256), scale=2.0)
    v = randn_bf16(rng, (rows, 8, 256))
    qw = oracle.f32_to_bf16(1.0 + 0.2 * rng.standard_normal(256).astype(np.float32))
    kw = oracle.f32_to_bf16(1.0 + 0.2 * rng.standard_normal(256).astype(np.float32))
    cos, sin = oracle.fill_rope_tables(256, 128, 10000.0, 256)
    pos = np.tile(np.arange(seq), batch)
    pos[1] = -1  # not prepared: its prepared rows keep their contents
    scale = 1 / 16
    out = empty_bf16((rows, QH, 256), dev)
    fill = 0x3F80
    qp = to_dev(np.full((rows, QH, 256), fill, np.uint16), dev)
    kp = to_dev(np.full((rows, 8, 256), fill, np.uint16), dev)
    vp = to_dev(np.full((rows, 8, 256), fill, np.uint16), dev)
    gk.check(gk.flash_attention_sliding_fwd_bf16_norm_rope(
        out, qp, kp, vp, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), to_dev(qw, dev),
        to_dev(kw, dev), to_dev(cos, dev), to_dev(sin, dev), to_dev(pos.astype(np.int32), dev),
        batch, seq, seq, window, scale), "sliding launcher")
    torch.cuda.synchronize()
    qph, kph, vph = from_dev_bf16(qp), from_dev_bf16(kp), from_dev_bf16(vp)
    assert np.all(qph.reshape(rows, -1)[1] == fill) and np.all(kph.reshape(rows, -1)[1] == fill)
    r = rows - 1
    c_row, s_row = cos[pos[r] * 128:(pos[r] + 1) * 128], sin[pos[r] * 128:(pos[r] + 1) * 128]
    exp_q = np.stack([oracle.prep_head(q[r, h], qw, c_row, s_row, 256) for h in range(QH)])
    _close_bits(qph.reshape(rows, QH, 256)[r], exp_q, "q_prepared")
    exp_k = np.stack([oracle.prep_head(k[r, h], kw, c_row, s_row, 256) for h in range(8)])
    _close_bits(kph.reshape(rows, 8, 256)[r], exp_k, "k_prepared")
    exp_v = np.stack([oracle.prep_head(v[r, h], None, None, None, 256) for h in range(8)])
    _close_bits(vph.reshape(rows, 8, 256)[r], exp_v, "v_prepared")
    exp = oracle.prefill_attention(qph.reshape(batch, seq, QH, 256), kph.reshape(batch, seq, 8, 256),
                                   vph.reshape(batch, seq, 8, 256), seq, seq, QH, 8, 256, window,
                                   scale, batch=batch)
    assert_close(from_dev_bf16(out).reshape(exp.shape), exp, f"sliding batch={batch} seq={seq}")


def test_launcher_argument_checks(dev):
    import torch
    z = torch.zeros(64, dtype=torch.int32, device=dev)
    args = [z] * 12
    # seqlen_q != seqlen_k, window <= 0, empty batch: invalid (src/gemma4_flash_attention_prefill.cu:1131-1138)
    assert gk.flash_attention_sliding_fwd_bf16_norm_rope(*args, 1, 4, 5, 8, 0.1) != 0
    assert gk.flash_attention_sliding_fwd_bf16_norm_rope(*args, 1, 4, 4, 0, 0.1) != 0
    assert gk.flash_attention_sliding_fwd_bf16_norm_rope(*args, 0, 4, 4, 8, 0.1) != 0
    assert gk.flash_attention_global_fwd_bf16_norm_rope(*([z] * 11), 1, 4, 5, 0.1) != 0
    nulls = [None] + [z] * 10
    assert gk.flash_attention_global_fwd_bf16_norm_rope(*nulls, 1, 4, 4, 0.1) != 0
    torch.cuda.synchronize()
