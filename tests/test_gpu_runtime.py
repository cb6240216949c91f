"""Runtime state on the GPU: the reference's own runtime test
(tests/test_runtime_state.cu:29-140) through the C-ABI, plus a ring walk
checked against the oracle's page bookkeeping."""
import math

import numpy as np
import pytest

import gemma_kv as gk
from oracle import oracle

pytestmark = pytest.mark.gpu


def _device_i32(ptr, count):
    import torch
    out = torch.empty(count, dtype=torch.int32, device="cuda:0")
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so.7")  # the runtime torch already loaded (same soname)
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert hip.hipMemcpy(out.data_ptr(), ptr, count * 4, 3) == 0  # device to device
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _device_f32(ptr, count):
    return _device_i32(ptr, count).view(np.float32)


def test_prefill_decode_metadata(dev):
    rt = gk.Runtime(2, 66, 64)
    gk.check(rt.init_code)
    gk.check(rt.prepare_prefill(64))
    import torch
    torch.cuda.synchronize()
    sc = rt.scalars()
    assert sc["token_count"] == 128
    seq = _device_i32(rt.device_ptr("seq_lengths"), 2)
    tb = _device_i32(rt.device_ptr("token_batch"), 128)
    tp = _device_i32(rt.device_ptr("token_position"), 128)
    assert list(seq) == [64, 64]
    assert tb[63] == 0 and tp[63] == 63 and tb[64] == 1 and tp[64] == 0  # batch-major
    s_stride = rt.config(False).max_pages_per_seq
    g_stride = rt.config(True).max_pages_per_seq
    spt, gpt = rt.host("sliding_page_table"), rt.host("global_page_table")
    assert spt[0] >= 0 and spt[s_stride] >= 0 and gpt[0] >= 0 and gpt[g_stride] >= 0

    gk.check(rt.prepare_decode_step())
    torch.cuda.synchronize()
    seq = _device_i32(rt.device_ptr("seq_lengths"), 2)
    tb = _device_i32(rt.device_ptr("token_batch"), 2)
    tp = _device_i32(rt.device_ptr("token_position"), 2)
    dspt = _device_i32(rt.device_ptr("sliding_page_table"), spt.size)
    dgpt = _device_i32(rt.device_ptr("global_page_table"), gpt.size)
    assert list(seq) == [65, 65] and list(tb) == [0, 1] and list(tp) == [64, 64]
    assert dspt[1] == 1 and dgpt[1] == 1

    # A step with a sequence at max_seq_len is refused and mutates nothing.
    rt.set_host_seq_lengths([64, 66])
    before = {k: rt.host(k) for k in gk.Runtime.HOST}
    assert rt.prepare_decode_step() == gk.HIP_ERROR_INVALID_VALUE
    for k, v in before.items():
        assert np.array_equal(rt.host(k), v), k
    rt.close()


def test_rope_tables(dev):
    rt = gk.Runtime(1, 4, 4)
    gk.check(rt.init_code)
    import torch
    torch.cuda.synchronize()
    s_half, g_half = 128, 64
    scos = _device_f32(rt.device_ptr("sliding_cos"), 4 * s_half)
    ssin = _device_f32(rt.device_ptr("sliding_sin"), 4 * s_half)
    gcos = _device_f32(rt.device_ptr("global_cos"), 4 * g_half)
    assert abs(scos[s_half] - math.cos(1.0)) <= 1e-6
    assert abs(ssin[s_half] - math.sin(1.0)) <= 1e-6
    assert abs(gcos[g_half + 1] - math.cos(1_000_000.0 ** (-2.0 / 512))) <= 1e-6
    ref_c, ref_s = oracle.fill_rope_tables(4, s_half, 10000.0, 256)
    assert np.array_equal(scos, ref_c) and np.array_equal(ssin, ref_s)
    rt.close()


def test_ring_walk_matches_oracle_bookkeeping(dev):
    """Prefill 1000 tokens then 300 decode steps with page 16: the sliding
    ring (window 1024, 65 slots) wraps; every step's host tables equal the
    oracle's, and the device copies equal the host ones."""
    import torch
    rt = gk.Runtime(3, 1400, 16)
    gk.check(rt.init_code)
    gk.check(rt.prepare_prefill(1000))
    scfg, gcfg = rt.config(False), rt.config(True)
    assert scfg.window_size == 1024 and scfg.max_pages_per_seq == oracle.sliding_pages_per_sequence(1400, 16)
    o_spt = np.full(rt.host("sliding_page_table").size, -1, np.int32)
    o_ss = o_spt.copy()
    o_gpt = np.full(rt.host("global_page_table").size, -1, np.int32)
    o_gs = o_gpt.copy()
    for b in range(3):
        assert oracle.ensure_range(o_spt, o_ss, scfg, b, 0, 1000) == 0
        assert oracle.ensure_range(o_gpt, o_gs, gcfg, b, 0, 1000) == 0
    for step in range(300):
        gk.check(rt.prepare_decode_step())
        for b in range(3):
            oracle.ensure_page(o_spt, o_ss, scfg, b, 1000 + step)
            oracle.ensure_page(o_gpt, o_gs, gcfg, b, 1000 + step)
        assert np.array_equal(rt.host("sliding_page_table"), o_spt)
        assert np.array_equal(rt.host("sliding_slot_logical_pages"), o_ss)
        assert np.array_equal(rt.host("global_page_table"), o_gpt)
    torch.cuda.synchronize()
    assert np.array_equal(_device_i32(rt.device_ptr("sliding_page_table"), o_spt.size), o_spt)
    assert np.array_equal(_device_i32(rt.device_ptr("global_page_table"), o_gpt.size), o_gpt)
    assert list(_device_i32(rt.device_ptr("seq_lengths"), 3)) == [1300] * 3
    rt.close()


def test_init_rejects_bad_sizes(dev):
    for args in [(0, 10, 4), (1, 0, 4), (1, 10, 0), (1, 262145, 64)]:
        assert gk.Runtime(*args).init_code == gk.HIP_ERROR_INVALID_VALUE


def _device_state(rt, batch):
    names = ("sliding_page_table", "global_page_table", "sliding_slot_logical_pages",
             "global_slot_logical_pages")
    out = {n: _device_i32(rt.device_ptr(n), rt.host(n).size) for n in names}
    out["seq_lengths"] = _device_i32(rt.device_ptr("seq_lengths"), batch)
    out["token_batch"] = _device_i32(rt.device_ptr("token_batch"), batch)
    out["token_position"] = _device_i32(rt.device_ptr("token_position"), batch)
    return out


def test_device_decode_step_matches_host_step(dev):
    """The device-side step (one kernel, no host bookkeeping) leaves exactly
    the device metadata the host step uploads, through a sliding-ring wrap
    (page 16, 65 slots), mixed with host steps; a refused device step (one
    step at max_seq_len) changes nothing and reports status 1."""
    import torch
    batch, max_seq = 3, 1200
    host_rt, dev_rt = gk.Runtime(batch, max_seq, 16), gk.Runtime(batch, max_seq, 16)
    gk.check(host_rt.init_code)
    gk.check(dev_rt.init_code)
    gk.check(host_rt.prepare_prefill(1000))
    gk.check(dev_rt.prepare_prefill(1000))
    for step in range(120):
        gk.check(host_rt.prepare_decode_step())
        if step % 40 == 39:
            gk.check(dev_rt.prepare_decode_step())  # host step after device steps: syncs first
        else:
            gk.check(dev_rt.prepare_decode_step_device())
        if step % 20 == 0 or step == 119:
            torch.cuda.synchronize()
            a, b = _device_state(host_rt, batch), _device_state(dev_rt, batch)
            for k in a:
                assert np.array_equal(a[k], b[k]), (step, k)
            assert dev_rt.device_step_status() == 0
    gk.check(dev_rt.sync_host())
    for k in gk.Runtime.HOST:
        if k in ("token_batch", "token_position"):
            assert np.array_equal(dev_rt.host(k)[:batch], host_rt.host(k)[:batch]), k
        else:
            assert np.array_equal(dev_rt.host(k), host_rt.host(k)), k
    # Refusal: sequence 1 at max_seq_len. Nothing changes, status 1.
    gk.check(dev_rt.prepare_prefill(max_seq - 5))  # rebuild, then walk up to max_seq_len
    for _ in range(5):
        gk.check(dev_rt.prepare_decode_step_device())
    torch.cuda.synchronize()
    assert dev_rt.device_step_status() == 0
    before = _device_state(dev_rt, batch)
    assert list(before["seq_lengths"]) == [max_seq] * batch
    gk.check(dev_rt.prepare_decode_step_device())
    torch.cuda.synchronize()
    assert dev_rt.device_step_status() == 1
    after = _device_state(dev_rt, batch)
    for k in before:
        assert np.array_equal(before[k], after[k]), k
    # The host form refuses the same step once it has synced.
    assert dev_rt.prepare_decode_step() == gk.HIP_ERROR_INVALID_VALUE
    host_rt.close()
    dev_rt.close()
