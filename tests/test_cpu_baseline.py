"""The timed CPU baseline (oracle/cpu_baseline.c) computes what the oracle
computes: the C config-1 loop equals the step-by-step oracle driven from
Python (ring bookkeeping, append, attention), for one thread and for a pool,
and the threaded layer-step equals oracle_decode_attention after the
reference append."""
import numpy as np

from oracle import oracle

HEADS, DIM, QH = 8, 256, 16


def test_config1_loop_matches_stepwise_oracle():
    steps, ring = 80, 32
    c = (1, ring, 1, ring, 1, HEADS, DIM, ring)
    q = oracle.fill_normal_bf16((steps, QH, DIM), 11)
    k = oracle.fill_normal_bf16((steps, HEADS, DIM), 12)
    v = oracle.fill_normal_bf16((steps, HEADS, DIM), 13)
    sec1, out1, ck1, cv1, pt1 = oracle.time_config1(q, k, v, c, 1 / 16, 1)
    sec4, out4, ck4, cv4, pt4 = oracle.time_config1(q, k, v, c, 1 / 16, 4)
    assert sec1 > 0 and sec4 > 0
    assert np.array_equal(out1, out4) and np.array_equal(ck1, ck4) and np.array_equal(cv1, cv4)

    exp_k = np.zeros(ring * HEADS * DIM, np.uint16)
    exp_v = np.zeros_like(exp_k)
    pt = np.full(ring, -1, np.int32)
    slots = np.full(ring, -1, np.int32)
    for t in range(steps):
        assert oracle.ensure_page(pt, slots, c, 0, t) >= 0
        oracle.kv_cache_write(exp_k, exp_v, c, pt, [0], [t], 0, k[t:t + 1], v[t:t + 1])
        exp = oracle.decode_attention(q[t:t + 1], exp_k, exp_v, pt, [t + 1], c, 0, 1 / 16)
        assert np.array_equal(out1[t], exp[0]), t
    assert np.array_equal(ck1, exp_k) and np.array_equal(cv1, exp_v)
    assert np.array_equal(pt1, pt)


def test_time_decode_layer_matches_oracle_on_ragged_batch():
    rng = np.random.default_rng(5)
    batch, page, max_pages = 3, 16, 8
    c = (2, batch * max_pages, page, max_pages, batch, HEADS, DIM, 0)
    seq = np.array([1, 77, 128], np.int32)
    pos = seq - 1
    pt = np.arange(batch * max_pages, dtype=np.int32)
    rows = c[0] * c[1] * page * HEADS * DIM
    ck = oracle.f32_to_bf16(rng.standard_normal(rows).astype(np.float32))
    cv = oracle.f32_to_bf16(rng.standard_normal(rows).astype(np.float32))
    q = oracle.f32_to_bf16(rng.standard_normal((batch, QH, DIM)).astype(np.float32))
    k = oracle.f32_to_bf16(rng.standard_normal((batch, HEADS, DIM)).astype(np.float32))
    v = oracle.f32_to_bf16(rng.standard_normal((batch, HEADS, DIM)).astype(np.float32))
    exp_k, exp_v = ck.copy(), cv.copy()
    oracle.kv_cache_write(exp_k, exp_v, c, pt, list(range(batch)), pos, 1, k, v)
    exp = oracle.decode_attention(q, exp_k, exp_v, pt, seq, c, 1, 1 / 16)
    for threads in (1, 5):
        gk, gv = ck.copy(), cv.copy()
        out = np.zeros_like(q)
        sec = oracle.time_decode_layer(out, q, gk, gv, pt, seq, pos, k, v, c, 1, 1 / 16, threads)
        assert sec > 0
        assert np.array_equal(out, exp) and np.array_equal(gk, exp_k) and np.array_equal(gv, exp_v)


def test_fill_normal_is_seeded_standard_normal():
    a = oracle.fill_normal_bf16((1 << 21,), 3, threads=1)
    b = oracle.fill_normal_bf16((1 << 21,), 3, threads=6)
    assert np.array_equal(a, b)
    x = oracle.bf16_to_f32(a).astype(np.float64)
    assert abs(x.mean()) < 5e-3 and abs(x.std() - 1.0) < 5e-3
    # Tail mass of N(0,1): P(|x| > 2) = 0.0455.
    assert abs((np.abs(x) > 2).mean() - 0.0455) < 2e-3
