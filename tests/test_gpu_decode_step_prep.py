"""Parity of the persistent decode step from raw projections
(gemma4_decode_step_layers_prep_bf16) against the oracle chain applied layer
by layer: prep_head on every query head and on the new K (learned RMSNorm +
split-half RoPE at the token's position) and V (scale-free RMSNorm; the
1 x 512 geometry derives it from the raw K), the append, then the attention.
The sum of squares is reduced in another order on the GPU, so a prepared
cache value may differ from the oracle's by one bf16 ulp (anything larger
fails, every untouched row is exact); attention outputs within max_abs 2e-2 /
max_rel 1e-2 of the oracle's on its own prepared rows."""
import math

import numpy as np
import pytest

import gemma_kv as gk
from kvtest import (assert_close, cache_config, fill_page_table, from_dev_bf16, randn_bf16,
                    ring_pages, to_dev)
from oracle import oracle

pytestmark = pytest.mark.gpu

HEADS, DIM = 8, 256


def is_global(layer):
    return layer == 47 or (layer + 1) % 6 == 0


def _ulp_diff(a_bits, b_bits):
    a = a_bits.astype(np.int32)
    b = b_bits.astype(np.int32)
    a = np.where(a & 0x8000, 0x8000 - (a & 0x7FFF), a + 0x8000)
    b = np.where(b & 0x8000, 0x8000 - (b & 0x7FFF), b + 0x8000)
    return np.abs(a - b)


def _workspace(dev, batch):
    import torch
    ws = torch.empty(gk.decode_step_workspace_bytes(batch) // 4, dtype=torch.int32, device=dev)
    gk.check(gk.decode_step_workspace_init(ws, batch), "workspace_init")
    return ws


CASES = [
    # first_layer, layer_count, seq_lengths, window, sliding page, global page, 1x512 globals
    (0, 7, [151], 64, 1, 16, False),        # ring wrapped; sliding, global, sliding
    (3, 9, [40, 9, 513], 256, 16, 16, False),  # batch 3, globals 5 and 11, ragged
    (44, 4, [300, 77], 128, 1, 64, False),  # batch 2, ends at the last (global) layer
    (0, 7, [151], 64, 1, 16, True),         # reference geometry: 1 x 512 global layer 5
    (3, 9, [40, 9, 513], 256, 16, 16, True),
]


@pytest.mark.parametrize("first,count,seq,window,s_page,g_page,ref", CASES)
def test_step_with_prep_against_oracle_chain(dev, first, count, seq, window, s_page, g_page,
                                             ref):
    import torch
    print(f"step+prep case first={first} count={count} seq={seq} ref={ref}", flush=True)
    rng = np.random.default_rng(sum(seq) + first + (1000 if ref else 0))
    batch = len(seq)
    layers = list(range(first, first + count))
    g_heads, g_dim = (1, 512) if ref else (HEADS, DIM)
    g_rot = 128 if ref else DIM
    n_s = sum(1 for l in range(48) if not is_global(l))
    s_cfg = cache_config(n_s, batch, s_page, ring_pages(window, s_page), HEADS, DIM, window)
    g_cfg = cache_config(48 - n_s, batch, g_page, (max(seq) + g_page - 1) // g_page, g_heads,
                         g_dim, 0)
    s_pt, g_pt = fill_page_table(s_cfg, seq), fill_page_table(g_cfg, seq)
    caches = {
        "sk": randn_bf16(rng, (s_cfg[0] * s_cfg[1] * s_page, HEADS, DIM)),
        "sv": randn_bf16(rng, (s_cfg[0] * s_cfg[1] * s_page, HEADS, DIM)),
        "gk": randn_bf16(rng, (g_cfg[0] * g_cfg[1] * g_page, g_heads, g_dim)),
        "gv": randn_bf16(rng, (g_cfg[0] * g_cfg[1] * g_page, g_heads, g_dim)),
    }
    geo = [(g_heads, g_dim) if is_global(l) else (HEADS, DIM) for l in layers]
    qs = [randn_bf16(rng, (batch, 16, d)) for _, d in geo]
    ks = [randn_bf16(rng, (batch, h, d), scale=3.0) for h, d in geo]
    vs = [randn_bf16(rng, (batch, h, d)) for h, d in geo]
    qws = [oracle.f32_to_bf16(1.0 + 0.2 * rng.standard_normal(d).astype(np.float32))
           for _, d in geo]
    kws = [oracle.f32_to_bf16(1.0 + 0.2 * rng.standard_normal(d).astype(np.float32))
           for _, d in geo]
    max_pos = max(seq) + 1
    s_cos, s_sin = oracle.fill_rope_tables(max_pos, DIM // 2, 10000.0, DIM)
    g_cos, g_sin = oracle.fill_rope_tables(max_pos, g_rot // 2, 1_000_000.0, g_dim)
    pos = [n - 1 for n in seq]
    scale = 1 / math.sqrt(DIM)

    # Oracle chain, layer by layer.
    exp = {n: a.copy() for n, a in caches.items()}
    exp_out = []
    for i, layer in enumerate(layers):
        g = is_global(layer)
        heads, dim = geo[i]
        rot = g_rot if g else DIM
        cos, sin = (g_cos, g_sin) if g else (s_cos, s_sin)
        half = rot // 2
        qp = np.zeros_like(qs[i])
        kp = np.zeros_like(ks[i])
        vp = np.zeros_like(vs[i])
        for b, p in enumerate(pos):
            c_row, s_row = cos[p * half:(p + 1) * half], sin[p * half:(p + 1) * half]
            for h in range(16):
                qp[b, h] = oracle.prep_head(qs[i][b, h], qws[i], c_row, s_row, rot)
            for h in range(heads):
                kp[b, h] = oracle.prep_head(ks[i][b, h], kws[i], c_row, s_row, rot)
                vp[b, h] = oracle.prep_head(ks[i][b, h] if (g and ref) else vs[i][b, h], None,
                                            None, None, rot)
        cfg, pt = (g_cfg, g_pt) if g else (s_cfg, s_pt)
        ck, cv = (exp["gk"], exp["gv"]) if g else (exp["sk"], exp["sv"])
        cl = oracle.layer_index(layer, g)
        oracle.kv_cache_write(ck, cv, cfg, pt, list(range(batch)), pos, cl, kp, vp)
        exp_out.append(oracle.decode_attention(qp, ck, cv, pt, seq, cfg, cl, scale))

    flat = lambda arrs: np.concatenate([a.reshape(-1) for a in arrs])
    d = {n: to_dev(a, dev) for n, a in caches.items()}
    ws = _workspace(dev, batch)
    total = sum(batch * 16 * w for _, w in geo)
    out = torch.zeros((total,), dtype=torch.int16, device=dev)
    gk.check(gk.decode_step_layers_prep_bf16(
        out, to_dev(flat(qs), dev), to_dev(flat(ks), dev), to_dev(flat(vs), dev), d["sk"],
        d["sv"], to_dev(s_pt, dev), gk.make_config(*s_cfg), d["gk"], d["gv"], to_dev(g_pt, dev),
        gk.make_config(*g_cfg), to_dev(np.asarray(seq, np.int32), dev),
        to_dev(np.asarray(pos, np.int32), dev), to_dev(flat(qws), dev), to_dev(flat(kws), dev),
        to_dev(s_cos, dev), to_dev(s_sin, dev), to_dev(g_cos, dev), to_dev(g_sin, dev),
        first, count, scale, batch, ws), "decode_step_layers_prep")
    torch.cuda.synchronize()
    assert gk.decode_step_status(ws) == 0
    for n in caches:
        got = from_dev_bf16(d[n]).reshape(caches[n].shape)
        changed = np.any(exp[n] != caches[n], axis=tuple(range(1, exp[n].ndim)))
        assert np.array_equal(got[~changed], caches[n][~changed]), n
        diff = _ulp_diff(got[changed], exp[n][changed])
        assert diff.max(initial=0) <= 1, f"{n}: max ulp diff {diff.max()}"
        assert (diff > 0).mean() < 0.02, f"{n}: {(diff > 0).mean():.3%} values differ"
    flat_out = from_dev_bf16(out)
    off = 0
    for i, (_, w) in enumerate(geo):
        got_i = flat_out[off:off + batch * 16 * w].reshape(batch, 16, w)
        off += batch * 16 * w
        assert_close(got_i, exp_out[i], f"layer {layers[i]}")


def test_step_with_prep_rejects_missing_tables(dev):
    import torch
    ws = _workspace(dev, 1)
    buf = torch.zeros(1 << 16, dtype=torch.int16, device=dev)
    i32 = torch.zeros(8, dtype=torch.int32, device=dev)
    f32 = torch.zeros(1 << 12, dtype=torch.float32, device=dev)
    s_cfg = gk.make_config(*cache_config(40, 1, 1, 64, HEADS, DIM, 64))
    g_cfg = gk.make_config(*cache_config(8, 1, 16, 4, HEADS, DIM, 0))

    def call(**kw):
        a = dict(out=buf, q=buf, k=buf, v=buf, sliding_k=buf, sliding_v=buf,
                 sliding_page_table=i32, sliding_config=s_cfg, global_k=buf, global_v=buf,
                 global_page_table=i32, global_config=g_cfg, seq_lengths=i32,
                 token_position=i32, q_norm_weight=buf, k_norm_weight=buf, sliding_cos=f32,
                 sliding_sin=f32, global_cos=f32, global_sin=f32, first_layer=0,
                 layer_count=6, softmax_scale=0.0625, batch_count=1, workspace=ws)
        a.update(kw)
        return gk.decode_step_layers_prep_bf16(**a)

    assert call(q_norm_weight=None) == 1
    assert call(k_norm_weight=None) == 1
    assert call(sliding_cos=None) == 1
    assert call(global_sin=None) == 1           # layer 5 is global
    torch.cuda.synchronize()
