"""Parity of the persistent multi-layer decode step
(gemma4_decode_step_layers_bf16) against the CPU oracle applied layer by
layer (append, then attend), and at the full BASELINE config-2 size against
the per-layer fused append+decode entry point. Appends are bit-exact;
attention outputs within max_abs 2e-2 / max_rel 1e-2."""
import math

import numpy as np
import pytest

import gemma_kv as gk
from kvtest import (assert_close, cache_config, empty_bf16, fill_page_table,
                    from_dev_bf16, randn_bf16, ring_pages, to_dev)
from oracle import oracle

pytestmark = pytest.mark.gpu

HEADS, DIM = 8, 256


def is_global(layer):
    return layer == 47 or (layer + 1) % 6 == 0


def _workspace(dev, batch):
    import torch
    nbytes = gk.decode_step_workspace_bytes(batch)
    assert nbytes > 0
    ws = torch.empty(nbytes // 4, dtype=torch.int32, device=dev)
    gk.check(gk.decode_step_workspace_init(ws, batch), "workspace_init")
    return ws


def _case(rng, first_layer, layer_count, seq, window, s_page, g_page):
    batch = len(seq)
    layers = list(range(first_layer, first_layer + layer_count))
    n_s = sum(1 for l in range(48) if not is_global(l))
    n_g = 48 - n_s
    s_max = ring_pages(window, s_page)
    g_max = (max(seq) + g_page - 1) // g_page
    s_cfg = cache_config(n_s, batch, s_page, s_max, HEADS, DIM, window)
    g_cfg = cache_config(n_g, batch, g_page, g_max, HEADS, DIM, 0)
    s_pt = fill_page_table(s_cfg, seq)
    g_pt = fill_page_table(g_cfg, seq)
    caches = {
        "sk": randn_bf16(rng, (s_cfg[0] * s_cfg[1] * s_page, HEADS, DIM)),
        "sv": randn_bf16(rng, (s_cfg[0] * s_cfg[1] * s_page, HEADS, DIM)),
        "gk": randn_bf16(rng, (g_cfg[0] * g_cfg[1] * g_page, HEADS, DIM)),
        "gv": randn_bf16(rng, (g_cfg[0] * g_cfg[1] * g_page, HEADS, DIM)),
    }
    q = randn_bf16(rng, (layer_count, batch, 16, DIM))
    k = randn_bf16(rng, (layer_count, batch, HEADS, DIM))
    v = randn_bf16(rng, (layer_count, batch, HEADS, DIM))
    return layers, s_cfg, g_cfg, s_pt, g_pt, caches, q, k, v


def _expected(layers, s_cfg, g_cfg, s_pt, g_pt, caches, q, k, v, seq, pos, scale):
    exp = {n: a.copy() for n, a in caches.items()}
    outs = []
    batch = len(seq)
    for i, layer in enumerate(layers):
        g = is_global(layer)
        cfg, pt = (g_cfg, g_pt) if g else (s_cfg, s_pt)
        ck, cv = (exp["gk"], exp["gv"]) if g else (exp["sk"], exp["sv"])
        cl = oracle.layer_index(layer, g)
        oracle.kv_cache_write(ck, cv, cfg, pt, list(range(batch)), pos, cl, k[i], v[i])
        outs.append(oracle.decode_attention(q[i], ck, cv, pt, seq, cfg, cl, scale))
    return exp, np.stack(outs)


def _run_step(dev, ws, layers, s_cfg, g_cfg, s_pt, g_pt, dcaches, q, k, v, seq, pos, scale,
              expect_status=0, fill=0):
    import torch
    batch = len(seq)
    out = empty_bf16((len(layers), batch, 16, DIM), dev)
    out.fill_(fill)
    code = gk.decode_step_layers_bf16(
        out, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), dcaches["sk"], dcaches["sv"],
        to_dev(s_pt, dev), gk.make_config(*s_cfg), dcaches["gk"], dcaches["gv"],
        to_dev(g_pt, dev), gk.make_config(*g_cfg), to_dev(np.asarray(seq, np.int32), dev),
        to_dev(np.asarray(pos, np.int32), dev), layers[0], len(layers), scale, batch, ws)
    gk.check(code, "decode_step")
    torch.cuda.synchronize()
    assert gk.decode_step_status(ws) == expect_status
    return from_dev_bf16(out)


STEP_CASES = [
    # first_layer, layer_count, seq_lengths, window, sliding page, global page
    (0, 7, [151], 64, 1, 16),          # ring wrapped, 5 sliding + global + sliding
    (3, 4, [40], 64, 4, 16),           # window not yet full, page-4 ring
    (0, 12, [9], 1024, 1, 64),         # fewer keys than splits: empty splits
    (44, 4, [300, 77], 128, 1, 64),    # batch 2, ends at the last (global) layer
    (5, 1, [1], 1024, 1, 64),          # one global layer, first token
    (0, 6, [2000, 1, 513], 256, 16, 64),  # batch 3 (10 splits per unit), ragged
    (3, 9, [3000, 1, 513, 64, 1024, 2, 700, 9], 1024, 16, 64),  # batch 8: 4 splits per unit
]


@pytest.mark.parametrize("first,count,seq,window,s_page,g_page", STEP_CASES)
def test_decode_step_against_oracle(dev, first, count, seq, window, s_page, g_page):
    rng = np.random.default_rng(sum(seq) + first * 7 + count)
    layers, s_cfg, g_cfg, s_pt, g_pt, caches, q, k, v = _case(
        rng, first, count, seq, window, s_page, g_page)
    pos = [n - 1 for n in seq]
    scale = 1 / math.sqrt(DIM)
    exp_caches, exp_out = _expected(layers, s_cfg, g_cfg, s_pt, g_pt, caches, q, k, v, seq,
                                    pos, scale)
    dcaches = {n: to_dev(a, dev) for n, a in caches.items()}
    ws = _workspace(dev, len(seq))
    got = _run_step(dev, ws, layers, s_cfg, g_cfg, s_pt, g_pt, dcaches, q, k, v, seq, pos,
                    scale)
    for n in caches:
        assert np.array_equal(from_dev_bf16(dcaches[n]).reshape(caches[n].shape),
                              exp_caches[n]), n
    for i, layer in enumerate(layers):
        assert_close(got[i], exp_out[i], f"layer {layer}")
    # Same workspace again (next epoch): the appended rows are already in
    # place, so the same step gives the same outputs.
    again = _run_step(dev, ws, layers, s_cfg, g_cfg, s_pt, g_pt, dcaches, q, k, v, seq, pos,
                      scale)
    assert np.array_equal(again, got)


REF_CASES = [
    # first_layer, layer_count, seq_lengths, window, sliding page, global page
    (0, 7, [151], 64, 1, 16),             # sliding run, 1x512 global layer 5, sliding 6
    (44, 4, [300, 77], 128, 1, 64),       # batch 2, ends at the last (global) layer
    (5, 1, [1], 1024, 1, 64),             # one global layer, first token
    (3, 9, [40, 9, 513], 256, 16, 16),    # batch 3, globals 5 and 11, ragged
]


def _ref_case(rng, first, count, seq, window, s_page, g_page, g_layers=8):
    """Inputs and oracle results of a step in the reference model's geometry
    (sliding 8 x 256, global 1 x 512); q/k/v rows flattened layer by layer at
    each layer's width."""
    batch = len(seq)
    layers = list(range(first, first + count))
    n_s = sum(1 for l in range(48) if not is_global(l))
    n_g = g_layers
    s_max = ring_pages(window, s_page)
    g_max = (max(seq) + g_page - 1) // g_page
    s_cfg = cache_config(n_s, batch, s_page, s_max, HEADS, DIM, window)
    g_cfg = cache_config(n_g, batch, g_page, g_max, 1, 512, 0)
    s_pt = fill_page_table(s_cfg, seq)
    g_pt = fill_page_table(g_cfg, seq)
    caches = {
        "sk": randn_bf16(rng, (s_cfg[0] * s_cfg[1] * s_page, HEADS, DIM)),
        "sv": randn_bf16(rng, (s_cfg[0] * s_cfg[1] * s_page, HEADS, DIM)),
        "gk": randn_bf16(rng, (g_cfg[0] * g_cfg[1] * g_page, 1, 512)),
        "gv": randn_bf16(rng, (g_cfg[0] * g_cfg[1] * g_page, 1, 512)),
    }
    geo = [(1, 512) if is_global(l) else (HEADS, DIM) for l in layers]
    qs = [randn_bf16(rng, (batch, 16, d)) for _, d in geo]
    ks = [randn_bf16(rng, (batch, h, d)) for h, d in geo]
    vs = [randn_bf16(rng, (batch, h, d)) for h, d in geo]
    pos = [n - 1 for n in seq]
    scale = 1 / math.sqrt(DIM)
    exp = {n: a.copy() for n, a in caches.items()}
    exp_out = []
    for i, layer in enumerate(layers):
        g = is_global(layer)
        cfg, pt = (g_cfg, g_pt) if g else (s_cfg, s_pt)
        ck, cv = (exp["gk"], exp["gv"]) if g else (exp["sk"], exp["sv"])
        cl = oracle.layer_index(layer, g)
        oracle.kv_cache_write(ck, cv, cfg, pt, list(range(batch)), pos, cl, ks[i], vs[i])
        exp_out.append(oracle.decode_attention(qs[i], ck, cv, pt, seq, cfg, cl, scale))
    flat = lambda arrs: np.concatenate([a.reshape(-1) for a in arrs])
    return dict(layers=layers, geo=geo, s_cfg=s_cfg, g_cfg=g_cfg, s_pt=s_pt, g_pt=g_pt,
                caches=caches, q=flat(qs), k=flat(ks), v=flat(vs), seq=seq, pos=pos,
                scale=scale, exp=exp, exp_out=exp_out)


def _ref_run(dev, ws, c, d, expect_status=0, fill=0):
    """One step of a _ref_case on device caches `d`; returns the output rows
    as a list per layer ([batch][16][width])."""
    import torch
    batch = len(c["seq"])
    total = sum(batch * 16 * w for _, w in c["geo"])
    out = torch.full((total,), fill, dtype=torch.int16, device=dev)
    gk.check(gk.decode_step_layers_bf16(
        out, to_dev(c["q"], dev), to_dev(c["k"], dev), to_dev(c["v"], dev), d["sk"], d["sv"],
        to_dev(c["s_pt"], dev), gk.make_config(*c["s_cfg"]), d["gk"], d["gv"],
        to_dev(c["g_pt"], dev), gk.make_config(*c["g_cfg"]),
        to_dev(np.asarray(c["seq"], np.int32), dev), to_dev(np.asarray(c["pos"], np.int32), dev),
        c["layers"][0], len(c["layers"]), c["scale"], batch, ws), "decode_step 1x512")
    torch.cuda.synchronize()
    assert gk.decode_step_status(ws) == expect_status
    flat = from_dev_bf16(out)
    rows, off = [], 0
    for _, w in c["geo"]:
        rows.append(flat[off:off + batch * 16 * w].reshape(batch, 16, w))
        off += batch * 16 * w
    return rows


@pytest.mark.parametrize("first,count,seq,window,s_page,g_page", REF_CASES)
def test_decode_step_reference_global_geometry(dev, first, count, seq, window, s_page, g_page):
    """The reference model's own geometry (src/gemma4.h:17-21): sliding layers
    8 x 256, global layers 1 KV head x 512 (GQA 16). Rows of q/k/v/out are laid
    out layer by layer at each layer's width. Checked against the oracle
    applied layer by layer: caches bit-exact, outputs within tolerance; a
    second step on the same workspace gives the same outputs."""
    c = _ref_case(np.random.default_rng(sum(seq) * 3 + first + count), first, count, seq,
                  window, s_page, g_page)
    d = {n: to_dev(a, dev) for n, a in c["caches"].items()}
    ws = _workspace(dev, len(seq))
    first_rows = _ref_run(dev, ws, c, d)
    for n in c["caches"]:
        assert np.array_equal(from_dev_bf16(d[n]).reshape(c["caches"][n].shape), c["exp"][n]), n
    again = _ref_run(dev, ws, c, d)
    for i, layer in enumerate(c["layers"]):
        assert np.array_equal(again[i], first_rows[i]), f"layer {layer}"
        assert_close(first_rows[i], c["exp_out"][i], f"layer {layer}")


def test_decode_step_reference_geometry_long_global(dev):
    """A long 1 x 512 global context (17000 keys at batch 2) in the reference
    geometry: the persistent runs of sliding layers never read the global
    cache, so its length must not fail their split-length check; the global
    layer runs as its own fused append + split-K launch with the combine.
    Same results as the oracle."""
    c = _ref_case(np.random.default_rng(17), 3, 4, [17000, 5], 128, 1, 64, g_layers=1)
    d = {n: to_dev(a, dev) for n, a in c["caches"].items()}
    ws = _workspace(dev, 2)
    rows = _ref_run(dev, ws, c, d)
    for n in c["caches"]:
        assert np.array_equal(from_dev_bf16(d[n]).reshape(c["caches"][n].shape), c["exp"][n]), n
    for i, layer in enumerate(c["layers"]):
        assert_close(rows[i], c["exp_out"][i], f"layer {layer}")


def test_decode_step_failure_sticky_reference_geometry(dev):
    """Sticky failure with the 1 x 512 global geometry, where global layers run
    as separate launches between the persistent runs: a wait made to give up
    at layer 2 (fault injection, limit 20 us) fails the step; the global
    layer 5 and the persistent run after it then write zeros and append
    nothing (the global cache stays as it was); the next step on the
    workspace writes only zeros and leaves every cache untouched; after
    workspace_init the step is correct again."""
    import torch
    c = _ref_case(np.random.default_rng(512), 0, 7, [151], 64, 1, 16)
    d = {n: to_dev(a, dev) for n, a in c["caches"].items()}
    ws = _workspace(dev, 1)
    gk.check(gk.decode_step_inject_stall(ws, 2, 2000), "inject_stall")
    print("decode step 1x512: stalled launch", flush=True)
    got1 = _ref_run(dev, ws, c, d, expect_status=1, fill=0x1234)
    assert c["layers"][5] == 5 and c["geo"][5] == (1, 512)
    assert not got1[5].any() and not got1[6].any()
    assert np.array_equal(from_dev_bf16(d["gk"]).reshape(c["caches"]["gk"].shape),
                          c["caches"]["gk"])
    assert np.array_equal(from_dev_bf16(d["gv"]).reshape(c["caches"]["gv"].shape),
                          c["caches"]["gv"])
    snap = {n: t.clone() for n, t in d.items()}
    print("decode step 1x512: launch on the failed workspace", flush=True)
    got2 = _ref_run(dev, ws, c, d, expect_status=1, fill=0x1234)
    assert not any(r.any() for r in got2)
    for n in d:
        assert torch.equal(d[n], snap[n]), n
    gk.check(gk.decode_step_workspace_init(ws, 1), "workspace_init")
    d = {n: to_dev(a, dev) for n, a in c["caches"].items()}
    got3 = _ref_run(dev, ws, c, d)
    for n in c["caches"]:
        assert np.array_equal(from_dev_bf16(d[n]).reshape(c["caches"][n].shape), c["exp"][n]), n
    for i, layer in enumerate(c["layers"]):
        assert_close(got3[i], c["exp_out"][i], f"layer {layer}")


def test_decode_step_failure_is_reported_and_sticky(dev):
    """A bounded wait made to give up from the host (fault injection: at layer
    2 one workgroup waits for a word nothing sets, limit 20 us) while every
    kernel still exits normally. The launch reports status 1 (synchronous and
    stream-ordered reads agree) and the stalled workgroup's output chunk is
    zero in every layer; the next launch on the workspace writes only zeros
    and leaves the caches untouched; after workspace_init the same step is
    correct again."""
    import torch
    rng = np.random.default_rng(99)
    seq, first, count = [151], 0, 6
    layers, s_cfg, g_cfg, s_pt, g_pt, caches, q, k, v = _case(rng, first, count, seq, 64, 1, 16)
    pos = [n - 1 for n in seq]
    scale = 1 / math.sqrt(DIM)
    exp_caches, exp_out = _expected(layers, s_cfg, g_cfg, s_pt, g_pt, caches, q, k, v, seq,
                                    pos, scale)
    dcaches = {n: to_dev(a, dev) for n, a in caches.items()}
    ws = _workspace(dev, 1)
    gk.check(gk.decode_step_inject_stall(ws, 2, 2000), "inject_stall")
    print("decode step: stalled launch", flush=True)
    got1 = _run_step(dev, ws, layers, s_cfg, g_cfg, s_pt, g_pt, dcaches, q, k, v, seq, pos,
                     scale, expect_status=1, fill=0x1234)
    pinned = torch.zeros(1, dtype=torch.int32, pin_memory=True)
    gk.check(gk.decode_step_status_async(ws, pinned), "status_async")
    torch.cuda.synchronize()
    assert int(pinned[0]) == 1
    # XCD 0, ticket 0 serves KV head 0, split 0: it combines output chunk 0
    # (dims 0..7) of query heads 0 and 1.
    assert not got1[:, 0, 0:2, 0:8].any()
    snap = {n: t.clone() for n, t in dcaches.items()}
    print("decode step: launch on the failed workspace", flush=True)
    got2 = _run_step(dev, ws, layers, s_cfg, g_cfg, s_pt, g_pt, dcaches, q, k, v, seq, pos,
                     scale, expect_status=1, fill=0x1234)
    assert not got2.any()
    for n in dcaches:
        assert torch.equal(dcaches[n], snap[n]), n
    # Re-initialised: the stall is cleared and the step is correct again.
    gk.check(gk.decode_step_workspace_init(ws, 1), "workspace_init")
    got3 = _run_step(dev, ws, layers, s_cfg, g_cfg, s_pt, g_pt, dcaches, q, k, v, seq, pos,
                     scale)
    for n in caches:
        assert np.array_equal(from_dev_bf16(dcaches[n]).reshape(caches[n].shape),
                              exp_caches[n]), n
    for i, layer in enumerate(layers):
        assert_close(got3[i], exp_out[i], f"layer {layer}")


def test_decode_step_cooperative_launch_matches(dev):
    """The optional cooperative launch mode runs the same kernel: same outputs
    and caches as the ordinary launch, status 0."""
    rng = np.random.default_rng(31)
    first, count, seq, window, s_page, g_page = 0, 7, [151], 64, 1, 16
    layers, s_cfg, g_cfg, s_pt, g_pt, caches, q, k, v = _case(
        rng, first, count, seq, window, s_page, g_page)
    pos = [n - 1 for n in seq]
    scale = 1 / math.sqrt(DIM)
    ws = _workspace(dev, 1)
    results = []
    for coop in (False, True):
        dcaches = {n: to_dev(a, dev) for n, a in caches.items()}
        gk.check(gk.decode_step_set_cooperative(coop), "set_cooperative")
        try:
            got = _run_step(dev, ws, layers, s_cfg, g_cfg, s_pt, g_pt, dcaches, q, k, v, seq,
                            pos, scale)
        finally:
            gk.check(gk.decode_step_set_cooperative(False), "set_cooperative")
        results.append((got, {n: from_dev_bf16(t) for n, t in dcaches.items()}))
    assert np.array_equal(results[0][0], results[1][0])
    for n in caches:
        assert np.array_equal(results[0][1][n], results[1][1][n]), n
    assert gk.lib().gemma4_decode_step_set_cooperative(2) != 0


def test_decode_step_rejects_bad_arguments(dev):
    import torch
    rng = np.random.default_rng(1)
    layers, s_cfg, g_cfg, s_pt, g_pt, caches, q, k, v = _case(rng, 0, 2, [10], 64, 1, 16)
    ws = _workspace(dev, 1)
    out = empty_bf16((2, 1, 16, DIM), dev)
    d = {n: to_dev(a, dev) for n, a in caches.items()}
    seq = to_dev(np.asarray([10], np.int32), dev)
    pos = to_dev(np.asarray([9], np.int32), dev)
    args = [out, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), d["sk"], d["sv"],
            to_dev(s_pt, dev), gk.make_config(*s_cfg), d["gk"], d["gv"], to_dev(g_pt, dev),
            gk.make_config(*g_cfg), seq, pos]
    bad_geom = gk.make_config(*cache_config(40, 1, 1, 64, 1, 512, 64))
    assert gk.decode_step_layers_bf16(*args, 47, 2, 0.0625, 1, ws) != 0   # past layer 47
    assert gk.decode_step_layers_bf16(*args, 0, 2, 0.0, 1, ws) != 0       # scale
    assert gk.decode_step_layers_bf16(*args, 0, 2, 0.0625, 9, ws) != 0    # batch > 8
    bad = list(args)
    bad[7] = bad_geom
    assert gk.decode_step_layers_bf16(*bad, 0, 2, 0.0625, 1, ws) != 0     # sliding 1x512
    small = torch.empty(16, dtype=torch.int32, device=dev)
    assert gk.decode_step_layers_bf16(*args, 0, 2, 0.0625, 1, small) != 0  # workspace
    torch.cuda.synchronize()


def test_decode_step_config2_matches_per_layer_path(dev):
    """BASELINE config 2 at full size (48 layers, context 8192, sliding page 1,
    global page 64): the persistent step against 48 per-layer fused
    append+decode launches on a copy of the same caches."""
    import torch
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    seq_len, pos = 8193, 8192
    n_s, n_g = 40, 8
    s_cfg = cache_config(n_s, 1, 1, 1024, HEADS, DIM, 1024)
    g_pages = (seq_len + 63) // 64
    g_cfg = cache_config(n_g, 1, 64, g_pages, HEADS, DIM, 0)

    def rnd(shape):
        return torch.randn(shape, generator=gen, device=dev).bfloat16().view(torch.int16)

    caches = {"sk": rnd((n_s * 1024, HEADS, DIM)), "sv": rnd((n_s * 1024, HEADS, DIM)),
              "gk": rnd((n_g * g_pages * 64, HEADS, DIM)),
              "gv": rnd((n_g * g_pages * 64, HEADS, DIM))}
    ref_caches = {n: t.clone() for n, t in caches.items()}
    q, k, v = rnd((48, 1, 16, DIM)), rnd((48, 1, HEADS, DIM)), rnd((48, 1, HEADS, DIM))
    i32 = dict(dtype=torch.int32, device=dev)
    s_pt = torch.arange(1024, **i32)
    g_pt = torch.arange(g_pages, **i32)
    seq_t = torch.tensor([seq_len], **i32)
    pos_t = torch.tensor([pos], **i32)
    scale = 1 / 16
    ws = _workspace(dev, 1)
    out = torch.zeros((48, 1, 16, DIM), dtype=torch.int16, device=dev)
    gk.check(gk.decode_step_layers_bf16(
        out, q, k, v, caches["sk"], caches["sv"], s_pt, gk.make_config(*s_cfg), caches["gk"],
        caches["gv"], g_pt, gk.make_config(*g_cfg), seq_t, pos_t, 0, 48, scale, 1, ws),
        "decode_step")
    torch.cuda.synchronize()
    assert gk.decode_step_status(ws) == 0

    ref = torch.zeros_like(out)
    s_conf, g_conf = gk.make_config(*s_cfg), gk.make_config(*g_cfg)
    s_split, s_n = gk.decode_split_plan(s_conf, 1, 1024)
    g_split, g_n = gk.decode_split_plan(g_conf, 1, seq_len)
    n = max(s_n, g_n)
    pm = torch.empty(16 * n, device=dev)
    pl = torch.empty(16 * n, device=dev)
    pa = torch.empty(16 * n * DIM, device=dev)
    si = gi = 0
    for layer in range(48):
        if is_global(layer):
            conf, ck, cv, pt, cl, sp, ns = g_conf, ref_caches["gk"], ref_caches["gv"], g_pt, gi, g_split, g_n
            gi += 1
        else:
            conf, ck, cv, pt, cl, sp, ns = s_conf, ref_caches["sk"], ref_caches["sv"], s_pt, si, s_split, s_n
            si += 1
        gk.check(gk.flash_attention_append_decode_paged_bf16(
            ref[layer], pm, pl, pa, q[layer], ck, cv, pt, seq_t, pos_t, k[layer], v[layer],
            conf, cl, scale, sp, ns, 1), "per-layer")
    torch.cuda.synchronize()
    for name in caches:
        assert torch.equal(caches[name], ref_caches[name]), name
    got = out.view(torch.bfloat16).float()
    exp = ref.view(torch.bfloat16).float()
    diff = (got - exp).abs()
    denom = torch.maximum(torch.maximum(got.abs(), exp.abs()), torch.ones_like(got))
    assert float(diff.max()) <= 2e-2 and float((diff / denom).max()) <= 1e-2
    # A second step on the same workspace (the appended rows now in place).
    out2 = torch.zeros_like(out)
    gk.check(gk.decode_step_layers_bf16(
        out2, q, k, v, caches["sk"], caches["sv"], s_pt, s_conf, caches["gk"], caches["gv"],
        g_pt, g_conf, seq_t, pos_t, 0, 48, scale, 1, ws), "decode_step again")
    torch.cuda.synchronize()
    assert gk.decode_step_status(ws) == 0
    assert torch.equal(out2, out)


def test_decode_step_reference_geometry_rejects_before_any_launch(dev):
    """With 1 x 512 global layers the step is several launches; a bad argument
    of any of them is rejected before the first one, so nothing is appended
    and no output row is written. Case 1: first layer 5 (global) with a bad
    sliding config for layer 6. Case 2: a global config whose num_layers
    covers global layer 5 but not 11."""
    import torch
    c = _ref_case(np.random.default_rng(77), 5, 7, [151], 64, 1, 16)
    d = {n: to_dev(a, dev) for n, a in c["caches"].items()}
    ws = _workspace(dev, 1)
    total = sum(16 * w for _, w in c["geo"])
    out = torch.full((total,), 0x1234, dtype=torch.int16, device=dev)
    seq = to_dev(np.asarray(c["seq"], np.int32), dev)
    pos = to_dev(np.asarray(c["pos"], np.int32), dev)

    def call(s_cfg, g_cfg):
        return gk.decode_step_layers_bf16(
            out, to_dev(c["q"], dev), to_dev(c["k"], dev), to_dev(c["v"], dev), d["sk"],
            d["sv"], to_dev(c["s_pt"], dev), gk.make_config(*s_cfg), d["gk"], d["gv"],
            to_dev(c["g_pt"], dev), gk.make_config(*g_cfg), seq, pos, 5, 7, c["scale"], 1, ws)

    bad_sliding = list(c["s_cfg"])
    bad_sliding[6] = 128  # head_dim the persistent kernel does not serve
    short_global = list(c["g_cfg"])
    short_global[0] = 1   # global cache layer 1 (model layer 11) out of range
    for s_cfg, g_cfg in ((bad_sliding, c["g_cfg"]), (c["s_cfg"], short_global)):
        assert call(s_cfg, g_cfg) == gk.HIP_ERROR_INVALID_VALUE
        torch.cuda.synchronize()
        assert (out == 0x1234).all()
        for n in c["caches"]:
            assert np.array_equal(from_dev_bf16(d[n]).reshape(c["caches"][n].shape),
                                  c["caches"][n]), n
    assert gk.decode_step_status(ws) == 0


def test_decode_step_rejects_cache_layers_out_of_range(dev):
    """A cache config whose num_layers does not cover a layer of the step
    (8 x 256 global cache of one layer; layers 0..11 use global cache layers
    0 and 1) is rejected before the launch: no output written, caches as
    they were."""
    import torch
    rng = np.random.default_rng(5)
    layers, s_cfg, g_cfg, s_pt, g_pt, caches, q, k, v = _case(rng, 0, 12, [40], 64, 1, 16)
    short = list(g_cfg)
    short[0] = 1
    dcaches = {n: to_dev(a, dev) for n, a in caches.items()}
    ws = _workspace(dev, 1)
    out = empty_bf16((12, 1, 16, DIM), dev)
    out.fill_(0x1234)
    code = gk.decode_step_layers_bf16(
        out, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), dcaches["sk"], dcaches["sv"],
        to_dev(s_pt, dev), gk.make_config(*s_cfg), dcaches["gk"], dcaches["gv"],
        to_dev(g_pt, dev), gk.make_config(*short), to_dev(np.asarray([40], np.int32), dev),
        to_dev(np.asarray([39], np.int32), dev), 0, 12, 0.0625, 1, ws)
    assert code == gk.HIP_ERROR_INVALID_VALUE
    torch.cuda.synchronize()
    assert (out == 0x1234).all()
    for n in caches:
        assert np.array_equal(from_dev_bf16(dcaches[n]).reshape(caches[n].shape), caches[n]), n
