"""Attention output projection + post-attention RMSNorm + residual
(gemma4_attention_o_projection_post_norm_bf16, reference
src/gemma4_flash_attention_decode.cu:34-129) against the oracle:
residual_out within one bf16 ulp plus the fp32 summation error (the oracle
sums in float64, the GPU on MFMA in fp32), normed_out within the north-star
tolerance (and one ulp of the tail applied to the GPU's own residual), ffn_residual exact on the GPU's normed row,
and the closed forms the oracle tests pin (one-hot attention row selects a
weight element, exactly)."""
import numpy as np
import pytest

import gemma_kv as gk
from kvtest import assert_close, empty_bf16, from_dev_bf16, randn_bf16, to_dev
from oracle import oracle

pytestmark = pytest.mark.gpu

HIDDEN = 3840


def _ulp_diff(a_bits, b_bits):
    a = a_bits.astype(np.int32)
    b = b_bits.astype(np.int32)
    a = np.where(a & 0x8000, 0x8000 - (a & 0x7FFF), a + 0x8000)
    b = np.where(b & 0x8000, 0x8000 - (b & 0x7FFF), b + 0x8000)
    return np.abs(a - b)


def _inputs(seed, rows, width):
    rng = np.random.default_rng(seed)
    attn = randn_bf16(rng, (rows, width))
    w = randn_bf16(rng, (HIDDEN, width), scale=0.02)
    g = oracle.f32_to_bf16((1.0 + 0.1 * rng.standard_normal(HIDDEN)).astype(np.float32))
    x = randn_bf16(rng, (rows, HIDDEN))
    return attn, w, g, x


def _run(dev, attn, w, g, x, stream=None):
    import torch
    rows, width = attn.shape
    outs = [empty_bf16((rows, HIDDEN), dev) for _ in range(3)]
    gk.check(gk.attention_o_projection_post_norm_bf16(
        *outs, to_dev(attn, dev), to_dev(w, dev), to_dev(g, dev), to_dev(x, dev), rows, width),
        "o projection")
    torch.cuda.synchronize()
    return [from_dev_bf16(t) for t in outs]


@pytest.mark.parametrize("rows,width,seed", [(1, 4096, 1), (1, 8192, 2), (3, 4096, 3), (5, 8192, 4),
                                             (17, 4096, 5), (40, 8192, 6), (70, 4096, 7)])
def test_o_projection_matches_oracle(dev, rows, width, seed):
    attn, w, g, x = _inputs(seed, rows, width)
    print(f"o_projection rows={rows} width={width} seed={seed}", flush=True)
    res, normed, ffn = _run(dev, attn, w, g, x)
    eres, enormed, effn = oracle.attention_o_projection(attn, w, g, x)
    # Residual: one bf16 ulp of the float64 value, plus the fp32 summation
    # error (relative to sum |a w|, which a sum that cancels to near zero
    # makes large in ulps of the result).
    d = _ulp_diff(res, eres)
    assert (d > 0).mean() < 0.02, (d > 0).mean()
    a64 = np.abs(oracle.bf16_to_f32(attn).astype(np.float64))
    w64 = np.abs(oracle.bf16_to_f32(w).astype(np.float64))
    mag = a64 @ w64.T
    exp = oracle.bf16_to_f32(eres).astype(np.float64)
    err = np.abs(oracle.bf16_to_f32(res) - exp)
    ulp = np.maximum(np.abs(exp), 1e-30) * 2.0 ** -7
    assert np.all(err <= ulp + 2.0 ** -16 * mag), float((err - ulp).max())
    assert_close(normed, enormed, "normed_out")
    # ffn_residual = x + normed cancels: a one-ulp step of normed (up to
    # 2^-6 at magnitude 2..4) can be most of a small sum, so it is checked
    # exactly against the GPU's own normed row below, not by tolerance.
    # The tail applied to the GPU's own residual row is the oracle's tail:
    # normed within one ulp, the residual add exact on the GPU's normed row.
    r32 = oracle.bf16_to_f32(res).astype(np.float64)
    scale = 1.0 / np.sqrt((r32 ** 2).mean(axis=1, keepdims=True) + 1e-6)
    n64 = r32 * scale * oracle.bf16_to_f32(g)
    assert _ulp_diff(normed, oracle.f32_to_bf16(n64.astype(np.float32))).max() <= 1
    s = oracle.bf16_to_f32(x).astype(np.float64) + oracle.bf16_to_f32(normed)
    assert np.array_equal(ffn, oracle.f32_to_bf16(s.astype(np.float32)))


@pytest.mark.parametrize("width", [4096, 8192])
def test_o_projection_one_hot_row_selects_weights(dev, width):
    rng = np.random.default_rng(9)
    w = randn_bf16(rng, (HIDDEN, width))
    g = np.full(HIDDEN, 0x3F80, np.uint16)
    x = np.zeros((2, HIDDEN), np.uint16)
    attn = np.zeros((2, width), np.uint16)
    attn[0, 5] = 0x3F80            # row 0 picks weight element 5 of every column
    attn[1, width - 1] = 0xBF80    # row 1 picks minus the last element
    res, normed, ffn = _run(dev, attn, w, g, x)
    assert np.array_equal(res[0], w[:, 5])
    assert np.array_equal(res[1], w[:, width - 1] ^ np.uint16(0x8000))
    assert np.array_equal(ffn, normed)


def test_o_projection_argument_checks(dev):
    import torch
    a = empty_bf16((1, 4096), dev)
    o = empty_bf16((1, HIDDEN), dev)
    w = empty_bf16((HIDDEN, 4096), dev)
    g = empty_bf16((HIDDEN,), dev)
    ok = 0
    assert gk.attention_o_projection_post_norm_bf16(o, o, o, a, w, g, o, 0, 4096) == ok
    assert gk.attention_o_projection_post_norm_bf16(o, o, o, a, w, g, o, 1, 2048) != ok
    assert gk.attention_o_projection_post_norm_bf16(o, o, o, a, w, g, o, -1, 4096) != ok
    assert gk.attention_o_projection_post_norm_bf16(None, o, o, a, w, g, o, 1, 4096) != ok
    torch.cuda.synchronize()
