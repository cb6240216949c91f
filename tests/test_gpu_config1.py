"""BASELINE config 1 on the GPU: one sliding layer (8 KV heads x 256, 16 query
heads, 1024-slot page-1 ring), 2048 sequential decode steps from an empty
cache, each appending one token then attending, q/k/v ~ N(0,1) from a seed,
scale 1/16.

The loop is the reference decode loop for one layer: the runtime's decode-step
bookkeeping (its device-side form, which maps the ring slot, writes the token
position and advances seq_len on the GPU, or the reference's host form with
its uploads) followed by the fused
append + split-K decode entry point, two launches per step, no host
synchronisation between steps. The oracle runs the same 2048 steps on the
CPU (ring bookkeeping, append, and the reference host attention of
tests/test_flash_attention.cu:124-172 applied to the step's query row).
Checked: the output of every 64th step (and the first four) within the
north-star tolerance, and the whole ring cache after the last step bit-exact."""
import math

import numpy as np
import pytest

import gemma_kv as gk
from kvtest import assert_close, device_i16, from_dev_bf16, randn_bf16, to_dev
from oracle import oracle

pytestmark = pytest.mark.gpu

HEADS, DIM, QH, WINDOW, STEPS = 8, 256, 16, 1024, 2048


def _checked(t):
    return t < 4 or t % 64 == 63 or t == STEPS - 1


@pytest.mark.parametrize("device_step", [True, False], ids=["device_step", "host_step"])
def test_config1_2048_sequential_steps(dev, device_step):
    import torch
    rng = np.random.default_rng(2048)
    q = randn_bf16(rng, (STEPS, 1, QH, DIM))
    k = randn_bf16(rng, (STEPS, 1, HEADS, DIM))
    v = randn_bf16(rng, (STEPS, 1, HEADS, DIM))
    scale = 1.0 / math.sqrt(DIM)

    rt = gk.Runtime(1, STEPS, 1)
    gk.check(rt.init_code, "runtime init")
    cfg = rt.config(False)
    assert cfg.as_tuple()[2:4] == (1, WINDOW)  # page 1, 1024 ring slots
    ck, cv = rt.device_ptr("sliding_cache_k"), rt.device_ptr("sliding_cache_v")
    pt, seq = rt.device_ptr("sliding_page_table"), rt.device_ptr("seq_lengths")
    pos = rt.device_ptr("token_position")
    split, n = gk.decode_split_plan(cfg, 1, WINDOW)
    pm = torch.empty(QH * n, device=dev)
    pl = torch.empty_like(pm)
    pa = torch.empty(QH * n * DIM, device=dev)
    dq, dk, dv = to_dev(q, dev), to_dev(k, dev), to_dev(v, dev)
    out = torch.zeros((STEPS, 1, QH, DIM), dtype=torch.int16, device=dev)
    row = QH * DIM * 2
    kv_row = HEADS * DIM * 2
    print(f"config1: {STEPS} steps, split {split} x {n}", flush=True)
    for t in range(STEPS):
        if device_step:
            gk.check(rt.prepare_decode_step_device(), f"device step {t}")
        else:
            gk.check(rt.prepare_decode_step(), f"host step {t}")
        gk.check(gk.flash_attention_append_decode_paged_bf16(
            out.data_ptr() + t * row, pm, pl, pa, dq.data_ptr() + t * row, ck, cv, pt, seq, pos,
            dk.data_ptr() + t * kv_row, dv.data_ptr() + t * kv_row, cfg, 0, scale, split, n, 1),
            f"append_decode step {t}")
    torch.cuda.synchronize()
    if device_step:
        assert rt.device_step_status() == 0
    got = from_dev_bf16(out)

    # Oracle: the same 2048 steps on the CPU.
    ocfg = (1, WINDOW, 1, WINDOW, 1, HEADS, DIM, WINDOW)
    exp_k = np.zeros((WINDOW, HEADS, DIM), np.uint16)
    exp_v = np.zeros_like(exp_k)
    o_pt = np.full(WINDOW, -1, np.int32)
    o_slots = np.full(WINDOW, -1, np.int32)
    checked = 0
    for t in range(STEPS):
        assert oracle.ensure_page(o_pt, o_slots, ocfg, 0, t) >= 0
        oracle.kv_cache_write(exp_k, exp_v, ocfg, o_pt, [0], [t], 0, k[t], v[t])
        if _checked(t):
            exp = oracle.decode_attention(q[t], exp_k, exp_v, o_pt, [t + 1], ocfg, 0, scale)
            assert_close(got[t], exp, f"step {t}")
            checked += 1
    assert checked == 4 + STEPS // 64

    # The ring after the last step: layer 0 of the runtime's sliding cache,
    # and the runtime's page table against the oracle's ring bookkeeping.
    rows = WINDOW * HEADS * DIM
    got_k = from_dev_bf16(device_i16(ck, rows, dev)).reshape(WINDOW, HEADS, DIM)
    got_v = from_dev_bf16(device_i16(cv, rows, dev)).reshape(WINDOW, HEADS, DIM)
    assert np.array_equal(got_k, exp_k)
    assert np.array_equal(got_v, exp_v)
    gk.check(rt.sync_host(), "sync_host")
    assert rt.host("sliding_page_table").tolist() == o_pt.tolist()
    assert rt.host("seq_lengths").tolist() == [STEPS]
    rt.close()
