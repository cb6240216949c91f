"""Parity of the persistent decode walk (gemma4_decode_walk_bf16: many
sequential decode steps of one layer in one launch) against the CPU oracle
run step by step (append at the step's position, then attend over the
window), including BASELINE config 1 in full through the runtime's walk
preparation. Appends and the final ring are bit-exact; attention outputs
within max_abs 2e-2 / max_rel 1e-2; the metadata the walk leaves equals what
as many single decode steps leave."""
import math

import numpy as np
import pytest

import gemma_kv as gk
from kvtest import (assert_close, cache_config, device_i16, empty_bf16, fill_page_table,
                    from_dev_bf16, randn_bf16, ring_pages, to_dev)
from oracle import oracle

pytestmark = pytest.mark.gpu

HEADS, DIM, QH = 8, 256, 16


def _workspace(dev, batch):
    import torch
    nbytes = gk.decode_step_workspace_bytes(batch)
    ws = torch.empty(nbytes // 4, dtype=torch.int32, device=dev)
    gk.check(gk.decode_step_workspace_init(ws, batch), "workspace_init")
    return ws


def _oracle_walk(ck, cv, cfg, pt, layer, seq0, q, k, v, scale, checked=None):
    """Steps t = 0..: append token t of every sequence at seq0[b] + t, then
    attend over seq0[b] + t + 1 keys (the reference's per-step loop)."""
    batch = len(seq0)
    outs = {}
    for t in range(q.shape[0]):
        pos = [int(s) + t for s in seq0]
        oracle.kv_cache_write(ck, cv, cfg, pt, list(range(batch)), pos, layer, k[t], v[t])
        if checked is None or checked(t):
            outs[t] = oracle.decode_attention(q[t], ck, cv, pt, [p + 1 for p in pos], cfg,
                                              layer, scale)
    return outs


# (batch, window (0 = global), page_size, seq0, steps, cache layers, layer)
CASES = [
    (1, 64, 4, [100], 40, 2, 1),          # ring wraps during the walk
    (2, 64, 1, [37, 200], 70, 1, 0),      # one sequence fills the ring, one wraps
    (4, 1024, 1, [1000, 3, 500, 1023], 24, 1, 0),  # 8 splits per unit
    (1, 0, 16, [50], 30, 3, 2),           # global cache, grows past a page
    (8, 32, 8, [0, 1, 2, 31, 32, 33, 64, 90], 12, 1, 0),  # from empty, 4 splits per unit
]


@pytest.mark.parametrize("case", CASES, ids=[f"b{c[0]}w{c[1]}p{c[2]}s{c[4]}" for c in CASES])
def test_walk_matches_oracle(dev, case):
    batch, window, page, seq0, steps, n_layers, layer = case
    print(f"walk case {case}", flush=True)
    rng = np.random.default_rng(7 + batch * 31 + steps)
    end = [s + steps for s in seq0]
    max_pages = ring_pages(window, page) if window > 0 else (max(end) + page - 1) // page
    cfg = cache_config(n_layers, batch, page, max_pages, HEADS, DIM, window)
    pt = fill_page_table(cfg, end)  # every position the walk appends is mapped
    rows = cfg[0] * cfg[1] * page
    ck = randn_bf16(rng, (rows, HEADS, DIM))
    cv = randn_bf16(rng, (rows, HEADS, DIM))
    q = randn_bf16(rng, (steps, batch, QH, DIM))
    k = randn_bf16(rng, (steps, batch, HEADS, DIM))
    v = randn_bf16(rng, (steps, batch, HEADS, DIM))
    scale = 1.0 / math.sqrt(DIM)

    exp_k, exp_v = ck.copy(), cv.copy()
    exp = _oracle_walk(exp_k, exp_v, cfg, pt, layer, seq0, q, k, v, scale)

    ws = _workspace(dev, batch)
    dck, dcv = to_dev(ck, dev), to_dev(cv, dev)
    seq_t = to_dev(np.asarray(seq0, np.int32), dev)
    pos_t = to_dev(np.full(batch, -7, np.int32), dev)
    out = empty_bf16((steps, batch, QH, DIM), dev)
    gk.check(gk.decode_walk_bf16(out, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), dck, dcv,
                                 to_dev(pt, dev), gk.make_config(*cfg), layer, seq_t, pos_t,
                                 steps, scale, batch, ws), "decode_walk")
    got = from_dev_bf16(out)
    assert gk.decode_step_status(ws) == 0
    for t in range(steps):
        assert_close(got[t], exp[t], f"step {t}")
    assert np.array_equal(from_dev_bf16(dck), exp_k)
    assert np.array_equal(from_dev_bf16(dcv), exp_v)
    assert seq_t.cpu().numpy().tolist() == end
    assert pos_t.cpu().numpy().tolist() == [e - 1 for e in end]


def test_walk_continues_across_launches(dev):
    """Two walks back to back on one workspace continue from the metadata the
    first one left; the result equals one walk of both halves' steps."""
    batch, window, page, steps = 2, 48, 2, 30
    seq0 = [10, 60]
    rng = np.random.default_rng(99)
    end = [s + 2 * steps for s in seq0]
    cfg = cache_config(1, batch, page, ring_pages(window, page), HEADS, DIM, window)
    pt = fill_page_table(cfg, end)
    rows = cfg[1] * page
    ck = randn_bf16(rng, (rows, HEADS, DIM))
    cv = randn_bf16(rng, (rows, HEADS, DIM))
    q = randn_bf16(rng, (2 * steps, batch, QH, DIM))
    k = randn_bf16(rng, (2 * steps, batch, HEADS, DIM))
    v = randn_bf16(rng, (2 * steps, batch, HEADS, DIM))
    scale = 0.0625
    exp_k, exp_v = ck.copy(), cv.copy()
    exp = _oracle_walk(exp_k, exp_v, cfg, pt, 0, seq0, q, k, v, scale)

    ws = _workspace(dev, batch)
    dck, dcv, dpt = to_dev(ck, dev), to_dev(cv, dev), to_dev(pt, dev)
    seq_t = to_dev(np.asarray(seq0, np.int32), dev)
    pos_t = to_dev(np.zeros(batch, np.int32), dev)
    dq, dk, dv = to_dev(q, dev), to_dev(k, dev), to_dev(v, dev)
    out = empty_bf16((2 * steps, batch, QH, DIM), dev)
    row = batch * QH * DIM * 2
    kv_row = batch * HEADS * DIM * 2
    for half in range(2):
        off = half * steps
        gk.check(gk.decode_walk_bf16(out.data_ptr() + off * row, dq.data_ptr() + off * row,
                                     dk.data_ptr() + off * kv_row, dv.data_ptr() + off * kv_row,
                                     dck, dcv, dpt, gk.make_config(*cfg), 0, seq_t, pos_t,
                                     steps, scale, batch, ws), f"walk half {half}")
    got = from_dev_bf16(out)
    for t in range(2 * steps):
        assert_close(got[t], exp[t], f"step {t}")
    assert np.array_equal(from_dev_bf16(dck), exp_k)
    assert seq_t.cpu().numpy().tolist() == end


def test_walk_rejects_bad_arguments(dev):
    import torch
    cfg = cache_config(1, 1, 1, 64, HEADS, DIM, 64)
    ws = _workspace(dev, 1)
    buf = torch.zeros(1 << 20, dtype=torch.int16, device=dev)
    i32 = torch.zeros(64, dtype=torch.int32, device=dev)
    c = gk.make_config(*cfg)
    bad = hipErrorInvalidValue = 1

    def call(**kw):
        a = dict(out=buf, q=buf, k=buf, v=buf, cache_k=buf, cache_v=buf, page_table=i32,
                 config=c, layer=0, seq_lengths=i32, token_position=i32, steps=4,
                 softmax_scale=0.0625, batch_count=1, workspace=ws)
        a.update(kw)
        return gk.decode_walk_bf16(**a)

    assert call(steps=0) == bad
    assert call(steps=65536) == bad
    assert call(layer=1) == bad
    assert call(softmax_scale=0.0) == bad
    assert call(batch_count=9) == bad
    assert call(config=gk.make_config(*cache_config(1, 1, 1, 64, 1, 512, 64))) == bad
    assert call(seq_lengths=None) == bad
    torch.cuda.synchronize()


def test_walk_config1_2048_steps(dev):
    """one sliding layer, 1024-slot page-1 ring, 2048
    sequential append+attend steps from an empty cache, as one walk prepared
    by the runtime; the ring, page table and lengths afterwards match the
    oracle's 2048 single steps."""
    steps = 2048
    rng = np.random.default_rng(2048)
    q = randn_bf16(rng, (steps, 1, QH, DIM))
    k = randn_bf16(rng, (steps, 1, HEADS, DIM))
    v = randn_bf16(rng, (steps, 1, HEADS, DIM))
    scale = 1.0 / math.sqrt(DIM)
    rt = gk.Runtime(1, steps, 1)
    gk.check(rt.init_code, "runtime init")
    cfg = rt.config(False)
    ck, cv = rt.device_ptr("sliding_cache_k"), rt.device_ptr("sliding_cache_v")
    pt, seq = rt.device_ptr("sliding_page_table"), rt.device_ptr("seq_lengths")
    pos = rt.device_ptr("token_position")
    gk.check(rt.prepare_decode_walk(steps), "prepare_decode_walk")
    ws = _workspace(dev, 1)
    out = empty_bf16((steps, 1, QH, DIM), dev)
    gk.check(gk.decode_walk_bf16(out, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), ck, cv,
                                 pt, cfg, 0, seq, pos, steps, scale, 1, ws), "decode_walk")
    got = from_dev_bf16(out)
    assert gk.decode_step_status(ws) == 0

    window = 1024
    ocfg = (1, window, 1, window, 1, HEADS, DIM, window)
    exp_k = np.zeros((window, HEADS, DIM), np.uint16)
    exp_v = np.zeros_like(exp_k)
    o_pt = np.full(window, -1, np.int32)
    o_slots = np.full(window, -1, np.int32)
    for t in range(steps):
        assert oracle.ensure_page(o_pt, o_slots, ocfg, 0, t) >= 0
        oracle.kv_cache_write(exp_k, exp_v, ocfg, o_pt, [0], [t], 0, k[t], v[t])
        if t < 4 or t % 64 == 63 or t == steps - 1:
            exp = oracle.decode_attention(q[t], exp_k, exp_v, o_pt, [t + 1], ocfg, 0, scale)
            assert_close(got[t], exp, f"step {t}")
    rows = window * HEADS * DIM
    assert np.array_equal(from_dev_bf16(device_i16(ck, rows, dev)).reshape(exp_k.shape), exp_k)
    assert np.array_equal(from_dev_bf16(device_i16(cv, rows, dev)).reshape(exp_v.shape), exp_v)
    gk.check(rt.sync_host(), "sync_host")
    assert rt.host("sliding_page_table").tolist() == o_pt.tolist()
    assert rt.host("seq_lengths").tolist() == [steps]
    assert rt.host("token_position").tolist()[:1] == [steps - 1]
    rt.close()
