"""Parity of the MFMA prefill-chunk attention against the CPU oracle (causal,
sliding window, prior context in the paged cache incl. a wrapped ring), and
at BASELINE config 5 size against an fp32 torch reference on the GPU."""
import math

import numpy as np
import pytest

import gemma_kv as gk
from kvtest import (assert_close, cache_config, empty_bf16, fill_page_table, from_dev_bf16,
                    randn_bf16, ring_pages, to_dev)
from oracle import oracle

pytestmark = pytest.mark.gpu
H, D = 8, 256
SLOT_BYTES = 256 + 2 * 130 * 256 * 4  # balanced-prefill workspace slot


def _full_keys(cache, cfg, pt, b, prior, chunk):
    """Contiguous keys [0, prior + Lq) of sequence b: cached prior keys read
    through the page table (zeros where unmapped or evicted), then the chunk."""
    num_layers, num_pages, page, max_pages, batch, heads, dim, window = cfg
    rows = cache.reshape(-1, heads, dim)
    out = np.zeros((prior + chunk.shape[0], heads, dim), np.uint16)
    for kp in range(prior):
        lp = kp // page
        phys = pt[b * max_pages + lp % max_pages]
        if phys < 0:
            continue
        out[kp] = rows[phys * page + kp % page]
    out[prior:] = chunk
    return out


@pytest.mark.parametrize("window,page,priors,lq", [
    (0, 16, None, 77),            # plain causal self-attention (reference launcher case)
    (32, 16, None, 100),          # sliding window, no prior
    (64, 4, [40, 150], 96),       # ring wrapped by the prior context, batch 2
    (0, 16, [100, 3], 70),        # global cache prior, ragged
    (0, 8, [0, 33], 65),          # one sequence with no prior
])
def test_prefill_chunk_matches_oracle(dev, window, page, priors, lq):
    rng = np.random.default_rng(lq + window)
    batch = 1 if priors is None else len(priors)
    scale = 1 / math.sqrt(D)
    q = randn_bf16(rng, (batch, lq, 16, D))
    k = randn_bf16(rng, (batch, lq, H, D))
    v = randn_bf16(rng, (batch, lq, H, D))
    out = empty_bf16((batch, lq, 16, D), dev)
    if priors is None:
        cfg = cache_config(1, 1, page, 4, H, D, window)
        gk.check(gk.flash_attention_prefill_chunk_paged_bf16(
            out, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), None, None, None, None,
            gk.make_config(*cfg), 0, batch, lq, scale))
        exp = oracle.prefill_attention(q, k, v, lq, lq, 16, H, D, window, scale, batch=batch)
    else:
        max_pages = ring_pages(window, page) if window else (max(priors) + page - 1) // page + 1
        cfg = cache_config(1, batch, page, max_pages, H, D, window)
        pt = fill_page_table(cfg, priors)
        ck = randn_bf16(rng, (batch * max_pages * page, H, D))
        cv = randn_bf16(rng, (batch * max_pages * page, H, D))
        gk.check(gk.flash_attention_prefill_chunk_paged_bf16(
            out, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), to_dev(ck, dev), to_dev(cv, dev),
            to_dev(pt, dev), to_dev(np.asarray(priors, np.int32), dev), gk.make_config(*cfg), 0,
            batch, lq, scale))
        exp = np.zeros((batch, lq, 16, D), np.uint16)
        for b, pr in enumerate(priors):
            kf = _full_keys(ck, cfg, pt, b, pr, k[b])
            vf = _full_keys(cv, cfg, pt, b, pr, v[b])
            exp[b] = oracle.prefill_attention(q[b:b + 1], kf[None], vf[None], lq, pr + lq, 16, H,
                                              D, window, scale)[0]
    import torch
    torch.cuda.synchronize()
    assert_close(from_dev_bf16(out), exp, f"prefill window={window} priors={priors}")


def _run_balanced(dev, rng, priors, lq, page, ws=None):
    """One global chunk through the balanced entry point and the plain one;
    returns both outputs, the oracle's and the workspace (reused when given)."""
    import torch
    batch = len(priors)
    scale = 1 / math.sqrt(D)
    q = randn_bf16(rng, (batch, lq, 16, D))
    k = randn_bf16(rng, (batch, lq, H, D))
    v = randn_bf16(rng, (batch, lq, H, D))
    max_pages = (max(priors) + page - 1) // page + 1
    cfg = cache_config(1, batch, page, max_pages, H, D, 0)
    pt = fill_page_table(cfg, priors)
    ck = randn_bf16(rng, (batch * max_pages * page, H, D))
    cv = randn_bf16(rng, (batch * max_pages * page, H, D))
    c = gk.make_config(*cfg)
    nbytes = gk.flash_attention_prefill_chunk_workspace_bytes(batch, lq, c)
    if ws is None:
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    assert ws.numel() >= nbytes
    args = [to_dev(x, dev) for x in (q, k, v, ck, cv, pt, np.asarray(priors, np.int32))]
    out_ws = empty_bf16((batch, lq, 16, D), dev)
    out_plain = empty_bf16((batch, lq, 16, D), dev)
    gk.check(gk.flash_attention_prefill_chunk_paged_bf16_ws(
        out_ws, *args, c, 0, batch, lq, scale, ws, ws.numel()), "balanced")
    gk.check(gk.flash_attention_prefill_chunk_paged_bf16(
        out_plain, *args, c, 0, batch, lq, scale), "plain")
    torch.cuda.synchronize()
    exp = np.zeros((batch, lq, 16, D), np.uint16)
    for b, pr in enumerate(priors):
        kf = _full_keys(ck, cfg, pt, b, pr, k[b])
        vf = _full_keys(cv, cfg, pt, b, pr, v[b])
        exp[b] = oracle.prefill_attention(q[b:b + 1], kf[None], vf[None], lq, pr + lq, 16, H, D,
                                          0, scale)[0]
    return from_dev_bf16(out_ws), from_dev_bf16(out_plain), exp, ws


@pytest.mark.parametrize("priors,lq,page", [
    ([0], 65, 16),          # two row blocks, too close to split
    ([0], 200, 16),         # four blocks: pairs (0, 3) split, (1, 2) not
    ([0], 130, 16),         # three blocks: the middle one unpaired
    ([100, 3], 321, 16),    # ragged priors, six blocks, a partial last block
    ([0, 33], 384, 8),      # one sequence with no prior
    ([700], 512, 64),       # prior longer than the chunk
])
def test_prefill_balanced_global_matches_oracle(dev, priors, lq, page):
    """The balanced global chunk (row blocks j and nb-1-j paired, the split
    block merged through the workspace) equals the oracle, and the plain
    kernel's output within the same tolerance; a second call on the same
    workspace with a smaller input checks that the arrival counters re-arm."""
    rng = np.random.default_rng(lq + sum(priors))
    got, plain, exp, ws = _run_balanced(dev, rng, priors, lq, page)
    assert_close(got, exp, f"balanced priors={priors} lq={lq}")
    assert_close(got, plain, f"balanced vs plain priors={priors} lq={lq}")
    got2, _, exp2, _ = _run_balanced(dev, rng, priors[:1], max(lq // 2, 65), page, ws)
    assert_close(got2, exp2, f"balanced second call priors={priors[:1]}")
    # Every slot's arrival counter (the first word of the slot) is re-armed to zero.
    slots = ws[: ws.numel() // SLOT_BYTES * SLOT_BYTES].view(-1, SLOT_BYTES)
    assert not slots[:, :4].any().item()


def test_prefill_balanced_workspace_shared_by_chunk_sizes(dev):
    """A workspace sized for the largest chunk serves a large, a small and
    again a large chunk: each slot keeps its place whatever the chunk
    length, so a small call's partials never land on a counter a larger
    call reads."""
    import torch
    rng = np.random.default_rng(77)
    cfg = gk.make_config(*cache_config(1, 1, 16, 33, H, D, 0))
    ws = torch.zeros(gk.flash_attention_prefill_chunk_workspace_bytes(1, 512, cfg),
                     dtype=torch.uint8, device=dev)
    for lq, prior in ((512, 0), (130, 40), (512, 9)):
        got, plain, exp, _ = _run_balanced(dev, rng, [prior], lq, 16, ws)
        assert_close(got, exp, f"shared workspace lq={lq}")
        assert_close(got, plain, f"shared workspace vs plain lq={lq}")


def test_prefill_balanced_argument_checks(dev):
    import torch
    cfg = gk.make_config(*cache_config(1, 1, 16, 4, H, D, 0))
    sliding = gk.make_config(*cache_config(1, 1, 16, 4, H, D, 32))
    lq = 256
    nbytes = gk.flash_attention_prefill_chunk_workspace_bytes(1, lq, cfg)
    # 2 pairs x 8 heads = 16 slots: a 256-byte counter + 2 halves x 130 x 256 floats each.
    assert nbytes == 16 * SLOT_BYTES
    assert gk.flash_attention_prefill_chunk_workspace_bytes(1, lq, sliding) == 0
    assert gk.flash_attention_prefill_chunk_workspace_bytes(1, 64, cfg) == 0  # one row block
    x = torch.zeros((1, lq, 16, D), dtype=torch.int16, device=dev)
    kv = torch.zeros((1, lq, H, D), dtype=torch.int16, device=dev)
    ws = torch.zeros(nbytes + 512, dtype=torch.uint8, device=dev)
    base = [x, x, kv, kv, None, None, None, None]
    bad = gk.HIP_ERROR_INVALID_VALUE
    assert gk.flash_attention_prefill_chunk_paged_bf16_ws(*base, cfg, 0, 1, lq, 0.1, None, 0) == bad
    assert gk.flash_attention_prefill_chunk_paged_bf16_ws(
        *base, cfg, 0, 1, lq, 0.1, ws, nbytes - 1) == bad
    assert gk.flash_attention_prefill_chunk_paged_bf16_ws(
        *base, cfg, 0, 1, lq, 0.1, ws.data_ptr() + 4, nbytes) == bad
    # Sliding chunks and single row blocks need no workspace.
    assert gk.flash_attention_prefill_chunk_paged_bf16_ws(*base, sliding, 0, 1, lq, 0.1, None, 0) == 0
    assert gk.flash_attention_prefill_chunk_paged_bf16_ws(*base, cfg, 0, 1, 64, 0.1, None, 0) == 0
    assert gk.flash_attention_prefill_chunk_paged_bf16_ws(*base, cfg, 0, 1, lq, 0.1, ws, nbytes) == 0
    torch.cuda.synchronize()


@pytest.mark.parametrize("layer_kind", ["sliding", "global", "global_balanced"])
def test_prefill_config5_full_size_against_torch_fp32(dev, layer_kind):
    """2048-row chunk; sliding (window 1024, page-1 ring of
    1024 slots holding the last 1024 of a 1536-token prior) or global (prior
    6144, page 64)."""
    import torch
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    lq = 2048
    if layer_kind == "sliding":
        window, page, prior = 1024, 1, 1536
        max_pages = 1024
    else:
        window, page, prior = 0, 64, 6144
        max_pages = (prior + lq) // page
    cfg = cache_config(1, 1, page, max_pages, H, D, window)
    pt = fill_page_table(cfg, [prior])
    rows = max_pages * page

    def rnd(shape):
        return torch.randn(shape, generator=gen, device=dev).bfloat16()
    ck, cv = rnd((rows, H, D)), rnd((rows, H, D))
    q, k, v = rnd((1, lq, 16, D)), rnd((1, lq, H, D)), rnd((1, lq, H, D))
    out = empty_bf16((1, lq, 16, D), dev)
    scale = 1 / 16
    args = [out, q.view(torch.int16), k.view(torch.int16), v.view(torch.int16),
            ck.view(torch.int16), cv.view(torch.int16), to_dev(pt, dev),
            to_dev(np.array([prior], np.int32), dev), gk.make_config(*cfg), 0, 1, lq, scale]
    if layer_kind == "global_balanced":
        nbytes = gk.flash_attention_prefill_chunk_workspace_bytes(1, lq, args[8])
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        gk.check(gk.flash_attention_prefill_chunk_paged_bf16_ws(*args, ws, nbytes))
    else:
        gk.check(gk.flash_attention_prefill_chunk_paged_bf16(*args))
    # fp32 reference: gather the visible prior keys through the ring, then the chunk.
    kpos = torch.arange(prior + lq, device=dev)
    lp = kpos // page
    phys = torch.as_tensor(pt, device=dev, dtype=torch.int64)[lp.clamp(max=prior - 1 if prior else 0) % max_pages]
    prow = phys * page + kpos % page
    kf = torch.cat([ck[prow[:prior]], k[0]]).float()    # [Lk, H, D]
    vf = torch.cat([cv[prow[:prior]], v[0]]).float()
    qpos = prior + torch.arange(lq, device=dev)
    mask = kpos[None, :] <= qpos[:, None]
    if window:
        mask &= kpos[None, :] > qpos[:, None] - window
    got = out.view(torch.bfloat16).float()[0]
    for kvh in range(H):
        qh = q[0, :, 2 * kvh:2 * kvh + 2].float().permute(1, 0, 2)  # [2, Lq, D]
        s = torch.einsum("gqd,kd->gqk", qh, kf[:, kvh]) * scale
        s = s.masked_fill(~mask, float("-inf"))
        o = torch.einsum("gqk,kd->gqd", torch.softmax(s, -1), vf[:, kvh])
        ref = o.permute(1, 0, 2).bfloat16().float()
        g = got[:, 2 * kvh:2 * kvh + 2]
        diff = (g - ref).abs()
        rel = diff / torch.maximum(torch.maximum(g.abs(), ref.abs()), torch.ones_like(g))
        assert diff.max().item() <= 2e-2 and rel.max().item() <= 1e-2, (kvh, diff.max().item())
