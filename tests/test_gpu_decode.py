"""Parity of the HIP split-K decode attention (and its fused-append form)
against the CPU oracle, within the north-star tolerance (max_abs 2e-2,
max_rel 1e-2 with denominator max(|a|,|b|,1)), and at full BASELINE sizes
against an fp32 torch reference plus size-independent properties."""
import math

import numpy as np
import pytest

import gemma_kv as gk
from kvtest import (assert_close, cache_config, empty_bf16, fill_page_table,
                    from_dev_bf16, randn_bf16, ring_pages, to_dev,
                    torch_decode_reference)
from oracle import oracle

pytestmark = pytest.mark.gpu


def _run_decode(dev, cfg, q, ck, cv, pt, seq, layer, scale, split_size, num_splits,
                fused=None, counters=None):
    import torch
    batch = len(seq)
    dim = cfg[6]
    out = empty_bf16((batch, 16, dim), dev)
    rows = batch * 16 * num_splits
    pm = torch.full((rows,), float("nan"), device=dev)
    pl = torch.full((rows,), float("nan"), device=dev)
    pa = torch.full((rows * dim,), float("nan"), device=dev)
    args = dict(config=gk.make_config(*cfg), layer=layer, softmax_scale=scale,
                split_size=split_size, num_splits=num_splits, batch_count=batch)
    if fused is None:
        code = gk.flash_attention_decode_paged_bf16(
            out, pm, pl, pa, to_dev(q, dev), ck, cv, to_dev(pt, dev),
            to_dev(np.asarray(seq, np.int32), dev), **args)
    else:
        pos, k_new, v_new = fused
        code = gk.flash_attention_append_decode_paged_bf16(
            out, pm, pl, pa, to_dev(q, dev), ck, cv, to_dev(pt, dev),
            to_dev(np.asarray(seq, np.int32), dev), to_dev(np.asarray(pos, np.int32), dev),
            to_dev(k_new, dev), to_dev(v_new, dev), split_counters=counters, **args)
    gk.check(code, "decode")
    torch.cuda.synchronize()
    return from_dev_bf16(out)


CASES = [
    # heads, dim, page, window, seq_lengths, split_size, num_splits
    (8, 256, 1, 1024, [1], 32, 1),
    (8, 256, 1, 1024, [33], 32, 2),
    (8, 256, 1, 1024, [1024], 32, 32),
    (8, 256, 1, 1024, [3000], 128, 8),          # ring wrapped
    (8, 256, 1, 1024, [1500], 1024, 1),         # single split, direct output
    (8, 256, 64, 1024, [2500, 77], 96, 11),     # page-64 ring, batch 2
    (8, 256, 64, 0, [4096, 1, 700], 256, 16),   # global, ragged batch
    (8, 256, 16, 0, [0, 513], 64, 9),           # empty sequence in a batch
    (8, 256, 1, 1024, [0], 32, 1),              # empty, direct zeros
    (8, 256, 64, 0, [2000], 20, 100),           # the reference split size 20
    (1, 512, 64, 0, [300, 4100], 128, 33),      # reference global geometry
    (1, 512, 64, 0, [65], 512, 1),
]


@pytest.mark.parametrize("heads,dim,page,window,seq,split_size,num_splits", CASES)
def test_decode_matches_oracle(dev, heads, dim, page, window, seq, split_size, num_splits):
    rng = np.random.default_rng(sum(seq) + split_size)
    batch = len(seq)
    max_pages = ring_pages(window, page) if window else (max(max(seq), 1) + page - 1) // page
    cfg = cache_config(2, batch, page, max_pages, heads, dim, window)
    pt = fill_page_table(cfg, seq)
    n_rows = 2 * batch * max_pages * page
    ck = randn_bf16(rng, (n_rows, heads, dim))
    cv = randn_bf16(rng, (n_rows, heads, dim))
    q = randn_bf16(rng, (batch, 16, dim))
    scale = 1.0 / math.sqrt(dim)
    exp = oracle.decode_attention(q, ck, cv, pt, seq, cfg, 1, scale)
    got = _run_decode(dev, cfg, q, to_dev(ck, dev), to_dev(cv, dev), pt, seq, 1, scale,
                      split_size, num_splits)
    assert_close(got, exp, f"seq={seq}")
    for b, n in enumerate(seq):
        if n == 0:
            assert not got[b].any()


def test_decode_huge_split_size(dev):
    """Splits past the live ones with split * split_size beyond int32: only
    split 0 holds keys, the others exit; the fused append lands and the output
    equals the oracle's."""
    rng = np.random.default_rng(21)
    heads, dim, page, window = 8, 256, 1, 1024
    seq = [1500]
    cfg = cache_config(1, 1, page, ring_pages(window, page), heads, dim, window)
    pt = fill_page_table(cfg, seq)
    rows = ring_pages(window, page) * page
    ck0 = randn_bf16(rng, (rows, heads, dim))
    cv0 = randn_bf16(rng, (rows, heads, dim))
    q = randn_bf16(rng, (1, 16, dim))
    k_new = randn_bf16(rng, (1, heads, dim))
    v_new = randn_bf16(rng, (1, heads, dim))
    pos = [seq[0] - 1]
    exp_k, exp_v = ck0.copy(), cv0.copy()
    oracle.kv_cache_write(exp_k, exp_v, cfg, pt, [0], pos, 0, k_new, v_new)
    exp = oracle.decode_attention(q, exp_k, exp_v, pt, seq, cfg, 0, 1 / 16)
    ck, cv = to_dev(ck0, dev), to_dev(cv0, dev)
    split_size, num_splits = 1 << 30, 8   # split 7 starts at 7 * 2^30 keys
    got = _run_decode(dev, cfg, q, ck, cv, pt, seq, 0, 1 / 16, split_size, num_splits,
                      fused=(pos, k_new, v_new))
    assert np.array_equal(from_dev_bf16(ck).reshape(exp_k.shape), exp_k)
    assert_close(got, exp, "huge split size")


def test_decode_skips_unmapped_pages(dev):
    rng = np.random.default_rng(11)
    heads, dim, page = 8, 256, 16
    seq = [900]
    cfg = cache_config(1, 1, page, 64, heads, dim, 0)
    pt = fill_page_table(cfg, seq)
    pt[[3, 17, 18]] = -1
    pt[40] = 10_000  # out-of-range physical page
    ck = randn_bf16(rng, (64 * page, heads, dim))
    cv = randn_bf16(rng, (64 * page, heads, dim))
    q = randn_bf16(rng, (1, 16, dim))
    exp = oracle.decode_attention(q, ck, cv, pt, seq, cfg, 0, 0.0625)
    got = _run_decode(dev, cfg, q, to_dev(ck, dev), to_dev(cv, dev), pt, seq, 0, 0.0625, 64, 15)
    assert_close(got, exp, "unmapped pages")


def test_decode_outlier_keys_max_tracking(dev):
    # 1% of keys scaled x8 (BASELINE long-context stress), many small splits.
    rng = np.random.default_rng(5)
    heads, dim, page = 8, 256, 64
    seq = [8192]
    cfg = cache_config(1, 1, page, 128, heads, dim, 0)
    pt = fill_page_table(cfg, seq)
    kf = rng.standard_normal((8192, heads, dim), dtype=np.float32)
    hot = rng.choice(8192, size=82, replace=False)
    kf[hot] *= 8.0
    ck = oracle.f32_to_bf16(kf)
    cv = randn_bf16(rng, (8192, heads, dim))
    q = randn_bf16(rng, (1, 16, dim))
    exp = oracle.decode_attention(q, ck, cv, pt, seq, cfg, 0, 1 / 16)
    got = _run_decode(dev, cfg, q, to_dev(ck, dev), to_dev(cv, dev), pt, seq, 0, 1 / 16, 128, 64)
    assert_close(got, exp, "outliers")


@pytest.mark.parametrize("heads,dim,page,window,seq_before,split_size,num_splits", [
    (8, 256, 1, 1024, 2047, 64, 16),   # ring slot reuse, new token in the last split
    (8, 256, 64, 1024, 130, 32, 5),
    (8, 256, 64, 0, 5000, 512, 10),
    (1, 512, 64, 0, 777, 64, 13),
    (8, 256, 1, 1024, 0, 32, 1),       # first token of a sequence
    # Full rings are split by ring slot in a combining launch. A ring whose
    # slots are exactly the window (page 16 x 64 pages here; ring_pages adds a
    # page for page sizes above 1) is full from 1024 keys on: the token's
    # slot 1500 % 1024 = 476 is owned by a split in the middle.
    (8, 256, -16, 1024, 1500, 16, 64),
    (8, 256, 1, 1024, 1023, 16, 64),   # the ring becomes full with this token
])
def test_fused_append_decode_equals_append_then_attend(dev, heads, dim, page, window,
                                                       seq_before, split_size, num_splits):
    rng = np.random.default_rng(seq_before + 3)
    batch = 2
    seq = [seq_before + 1, max(1, seq_before // 3 + 1)]
    exact_ring = page < 0   # a negative page size asks for a ring of exactly the window
    page = abs(page)
    max_pages = (window // page if exact_ring else ring_pages(window, page)) if window else \
        (max(seq) + page - 1) // page
    cfg = cache_config(1, batch, page, max_pages, heads, dim, window)
    pt = fill_page_table(cfg, seq)
    n_rows = batch * max_pages * page
    ck0 = randn_bf16(rng, (n_rows, heads, dim))
    cv0 = randn_bf16(rng, (n_rows, heads, dim))
    q = randn_bf16(rng, (batch, 16, dim))
    k_new = randn_bf16(rng, (batch, heads, dim))
    v_new = randn_bf16(rng, (batch, heads, dim))
    pos = [n - 1 for n in seq]
    exp_k, exp_v = ck0.copy(), cv0.copy()
    oracle.kv_cache_write(exp_k, exp_v, cfg, pt, list(range(batch)), pos, 0, k_new, v_new)
    exp = oracle.decode_attention(q, exp_k, exp_v, pt, seq, cfg, 0, 1 / math.sqrt(dim))
    ck, cv = to_dev(ck0, dev), to_dev(cv0, dev)
    got = _run_decode(dev, cfg, q, ck, cv, pt, seq, 0, 1 / math.sqrt(dim), split_size,
                      num_splits, fused=(pos, k_new, v_new))
    assert np.array_equal(from_dev_bf16(ck).reshape(exp_k.shape), exp_k)
    assert np.array_equal(from_dev_bf16(cv).reshape(exp_v.shape), exp_v)
    assert_close(got, exp, "fused")
    # The unfused kernel on the appended cache gives the same bits.
    unfused = _run_decode(dev, cfg, q, ck, cv, pt, seq, 0, 1 / math.sqrt(dim), split_size,
                          num_splits)
    assert np.array_equal(unfused, got)
    # In-kernel split combine (self-re-arming counters): same result on three
    # calls in a row, and the counters end at zero.
    import torch
    counters = torch.zeros(batch * heads, dtype=torch.int32, device=dev)
    for _ in range(3):
        again = _run_decode(dev, cfg, q, ck, cv, pt, seq, 0, 1 / math.sqrt(dim), split_size,
                            num_splits, fused=(pos, k_new, v_new), counters=counters)
        assert_close(again, exp, "fused, in-kernel combine")
        assert np.abs(oracle.bf16_to_f32(again) - oracle.bf16_to_f32(got)).max() <= 2 ** -7
    assert not counters.cpu().numpy().any()
    assert np.array_equal(from_dev_bf16(ck).reshape(exp_k.shape), exp_k)


@pytest.mark.parametrize("window,page", [(1024, 16), (0, 64)], ids=["ring", "global"])
def test_fused_append_to_unmapped_page(dev, window, page):
    """A token whose page is unmapped is not stored (the reference's write
    rule) and does not attend; the other sequence's token does both. The
    ring case is full, so its keys are split by ring slot."""
    rng = np.random.default_rng(77 + page)
    heads, dim = 8, 256
    seq = [1601, 900]
    batch = len(seq)
    max_pages = ring_pages(window, page) if window else (max(seq) + page - 1) // page
    cfg = cache_config(1, batch, page, max_pages, heads, dim, window)
    pt = fill_page_table(cfg, seq)
    pos = [n - 1 for n in seq]
    pt[0 * max_pages + (pos[0] // page) % max_pages] = -1   # sequence 0's token page
    n_rows = batch * max_pages * page
    ck0 = randn_bf16(rng, (n_rows, heads, dim))
    cv0 = randn_bf16(rng, (n_rows, heads, dim))
    q = randn_bf16(rng, (batch, 16, dim))
    k_new = randn_bf16(rng, (batch, heads, dim))
    v_new = randn_bf16(rng, (batch, heads, dim))
    exp_k, exp_v = ck0.copy(), cv0.copy()
    oracle.kv_cache_write(exp_k, exp_v, cfg, pt, list(range(batch)), pos, 0, k_new, v_new)
    exp = oracle.decode_attention(q, exp_k, exp_v, pt, seq, cfg, 0, 1 / 16)
    split, n = gk.decode_split_plan(gk.make_config(*cfg), batch, max(seq))
    ck, cv = to_dev(ck0, dev), to_dev(cv0, dev)
    got = _run_decode(dev, cfg, q, ck, cv, pt, seq, 0, 1 / 16, split, n,
                      fused=(pos, k_new, v_new))
    assert np.array_equal(from_dev_bf16(ck).reshape(exp_k.shape), exp_k)
    assert np.array_equal(from_dev_bf16(cv).reshape(exp_v.shape), exp_v)
    assert_close(got, exp, "unmapped token page")


D512_EDGES = [
    # seq_lengths, split_size, num_splits, unmapped pages, outliers
    ([8193], 64, 129, (), False),           # 64-key splits
    ([1000, 257], 256, 4, (), False),       # long splits, ragged batch
    ([4100], 512, 9, (5, 17, 30), False),   # unmapped pages inside splits
    ([8192], 128, 64, (), True),            # 1% of keys x8: the running maximum moves
    ([17], 16, 2, (), False),               # a split of one key
    ([3000], 1024, 3, (40,), False),        # splits longer than one 512-key row window
]


@pytest.mark.parametrize("seq,split_size,num_splits,holes,outliers", D512_EDGES)
def test_decode_1x512_edges(dev, seq, split_size, num_splits, holes, outliers):
    """Edge cases of the reference model's global geometry (1 KV head x 512,
    16 query heads): fused append of the last token against the oracle's
    append-then-attend, caches bit-exact and outputs within the north-star
    tolerance; the unfused call on the appended cache gives the same bits."""
    rng = np.random.default_rng(sum(seq) + split_size)
    heads, dim, page = 1, 512, 64
    batch = len(seq)
    max_pages = (max(seq) + page - 1) // page
    cfg = cache_config(1, batch, page, max_pages, heads, dim, 0)
    pt = fill_page_table(cfg, seq)
    for h in holes:
        pt[h] = -1
    n_rows = batch * max_pages * page
    kf = rng.standard_normal((n_rows, heads, dim), dtype=np.float32)
    if outliers:
        hot = rng.choice(n_rows, size=n_rows // 100, replace=False)
        kf[hot] *= 8.0
    ck0 = oracle.f32_to_bf16(kf)
    cv0 = randn_bf16(rng, (n_rows, heads, dim))
    q = randn_bf16(rng, (batch, 16, dim))
    k_new = randn_bf16(rng, (batch, heads, dim))
    v_new = randn_bf16(rng, (batch, heads, dim))
    pos = [n - 1 for n in seq]
    scale = 1 / math.sqrt(dim)
    exp_k, exp_v = ck0.copy(), cv0.copy()
    oracle.kv_cache_write(exp_k, exp_v, cfg, pt, list(range(batch)), pos, 0, k_new, v_new)
    exp = oracle.decode_attention(q, exp_k, exp_v, pt, seq, cfg, 0, scale)
    ck, cv = to_dev(ck0, dev), to_dev(cv0, dev)
    got = _run_decode(dev, cfg, q, ck, cv, pt, seq, 0, scale, split_size, num_splits,
                      fused=(pos, k_new, v_new))
    assert np.array_equal(from_dev_bf16(ck).reshape(exp_k.shape), exp_k)
    assert np.array_equal(from_dev_bf16(cv).reshape(exp_v.shape), exp_v)
    assert_close(got, exp, "1x512 fused")
    unfused = _run_decode(dev, cfg, q, ck, cv, pt, seq, 0, scale, split_size, num_splits)
    assert np.array_equal(unfused, got)


def test_split_count_invariance_closed_forms(dev):
    import torch
    rng = np.random.default_rng(99)
    heads, dim, page = 8, 256, 64
    seq = [3333]
    cfg = cache_config(1, 1, page, 64, heads, dim, 0)
    pt = fill_page_table(cfg, seq)
    ck = randn_bf16(rng, (64 * page, heads, dim))
    cv = randn_bf16(rng, (64 * page, heads, dim))
    q = randn_bf16(rng, (1, 16, dim))
    dck, dcv = to_dev(ck, dev), to_dev(cv, dev)
    outs = [oracle.bf16_to_f32(_run_decode(dev, cfg, q, dck, dcv, pt, seq, 0, 1 / 16, s, n))
            for s, n in [(3333, 1), (32, 105), (224, 15), (1024, 4)]]
    for o in outs[1:]:
        assert np.abs(o - outs[0]).max() <= 2 ** -7  # bf16 rounding of fp32-equal values
    # q = 0 -> uniform weights -> mean of the live V rows.
    zq = np.zeros_like(q)
    got = oracle.bf16_to_f32(_run_decode(dev, cfg, zq, dck, dcv, pt, seq, 0, 1 / 16, 256, 14))
    mean = oracle.bf16_to_f32(cv[:3333]).astype(np.float64).mean(axis=0)  # [heads, dim]
    expect = np.repeat(mean, 2, axis=0)
    assert np.abs(got[0] - expect).max() <= 2e-3
    torch.cuda.synchronize()


@pytest.mark.parametrize("case", ["config2_global_8192", "config4_131072_outliers",
                                  "config3_batch64_mixed"])
def test_full_size_against_torch_fp32(dev, case):
    """BASELINE sizes: HIP vs an fp32 torch reference of the same paged gather."""
    import torch
    gen = torch.Generator(device=dev)
    gen.manual_seed(2024)
    heads, dim, page = 8, 256, 64
    if case == "config2_global_8192":
        seq = [8192]
    elif case == "config4_131072_outliers":
        seq = [131072]
    else:
        rng = np.random.default_rng(64)
        seq = rng.integers(512, 32769, size=64).tolist()
    batch = len(seq)
    max_pages = (max(seq) + page - 1) // page
    cfg = cache_config(1, batch, page, max_pages, heads, dim, 0)
    pt = fill_page_table(cfg, seq)
    n_rows = batch * max_pages * page
    ck = torch.randn((n_rows, heads, dim), generator=gen, device=dev).bfloat16()
    if case == "config4_131072_outliers":
        hot = torch.randperm(n_rows, generator=gen, device=dev)[: n_rows // 100]
        ck[hot] *= 8
    cv = torch.randn((n_rows, heads, dim), generator=gen, device=dev).bfloat16()
    q = torch.randn((batch, 16, dim), generator=gen, device=dev).bfloat16()
    split_size, num_splits = gk.decode_split_plan(gk.make_config(*cfg), batch, max(seq))
    out = empty_bf16((batch, 16, dim), dev)
    rows = batch * 16 * num_splits
    pm = torch.empty(rows, device=dev)
    pl = torch.empty(rows, device=dev)
    pa = torch.empty(rows * dim, device=dev)
    ck_i, cv_i, q_i = ck.view(torch.int16), cv.view(torch.int16), q.view(torch.int16)
    gk.check(gk.flash_attention_decode_paged_bf16(
        out, pm, pl, pa, q_i, ck_i, cv_i, to_dev(pt, dev), to_dev(np.asarray(seq, np.int32), dev),
        gk.make_config(*cfg), 0, 1 / 16, split_size, num_splits, batch))
    ref = torch_decode_reference(q_i, ck_i, cv_i, pt, seq, cfg, 0, 1 / 16)
    got = out.view(torch.bfloat16).float()
    ref_b = ref.bfloat16().float()
    diff = (got - ref_b).abs()
    rel = diff / torch.maximum(torch.maximum(got.abs(), ref_b.abs()), torch.ones_like(got))
    assert diff.max().item() <= 2e-2 and rel.max().item() <= 1e-2, (diff.max().item(), rel.max().item())
    assert torch.isfinite(got).all()


def test_decode_error_convention(dev):
    cfg = gk.make_config(40, 1024, 1, 1024, 1, 8, 256, 1024)
    buf = empty_bf16(1 << 16, dev)
    idx = to_dev(np.zeros(1024, np.int32), dev)
    f = gk.flash_attention_decode_paged_bf16
    inval = gk.HIP_ERROR_INVALID_VALUE
    assert f(buf, None, None, None, buf, buf, buf, idx, idx, cfg, 0, 0.0625, 32, 1, 0) == 0
    assert f(buf, None, None, None, buf, buf, buf, idx, idx, cfg, 40, 0.0625, 32, 1, 1) == inval
    assert f(buf, None, None, None, buf, buf, buf, idx, idx, cfg, 0, 0.0, 32, 1, 1) == inval
    assert f(buf, None, None, None, buf, buf, buf, idx, idx, cfg, 0, 0.0625, 0, 1, 1) == inval
    assert f(buf, None, None, None, buf, buf, buf, idx, idx, cfg, 0, 0.0625, 32, 4, 1) == inval  # no partials
    assert f(buf, None, None, None, buf, buf, buf, idx, idx, cfg, 0, 0.0625, 32, 1, 2) == inval  # batch > batch_size
    small_ring = gk.make_config(40, 512, 1, 512, 1, 8, 256, 1024)  # capacity < window
    assert f(buf, None, None, None, buf, buf, buf, idx, idx, small_ring, 0, 0.0625, 32, 1, 1) == inval
    odd = gk.make_config(40, 1024, 1, 1024, 1, 4, 128, 1024)  # unsupported geometry
    assert f(buf, None, None, None, buf, buf, buf, idx, idx, odd, 0, 0.0625, 32, 1, 1) == inval


@pytest.mark.parametrize("heads,dim,page,window,seq,split_size,num_splits", [
    (8, 256, 1, 1024, [3000], 64, 16),
    (8, 256, 64, 0, [4096, 700], 256, 16),
    (1, 512, 64, 0, [300, 4100], 128, 33),
])
def test_split_and_combine_phases(dev, heads, dim, page, window, seq, split_size, num_splits):
    """Phase 1 partials match the oracle's split partials (m in natural-log
    units, l, unnormalised acc: the reference layout), and phase 2 reproduces
    the one-call result bit for bit."""
    import torch
    rng = np.random.default_rng(len(seq) * 17 + split_size)
    batch = len(seq)
    max_pages = ring_pages(window, page) if window else (max(seq) + page - 1) // page
    cfg = cache_config(1, batch, page, max_pages, heads, dim, window)
    pt = fill_page_table(cfg, seq)
    n_rows = batch * max_pages * page
    ck = randn_bf16(rng, (n_rows, heads, dim))
    cv = randn_bf16(rng, (n_rows, heads, dim))
    q = randn_bf16(rng, (batch, 16, dim))
    scale = 1 / math.sqrt(dim)
    c = gk.make_config(*cfg)
    rows = batch * 16 * num_splits
    pm = torch.full((rows,), float("nan"), device=dev)
    pl = torch.full((rows,), float("nan"), device=dev)
    pa = torch.full((rows * dim,), float("nan"), device=dev)
    out = empty_bf16((batch, 16, dim), dev)
    dq, dck, dcv = to_dev(q, dev), to_dev(ck, dev), to_dev(cv, dev)
    dpt, dseq = to_dev(pt, dev), to_dev(np.asarray(seq, np.int32), dev)
    gk.check(gk.flash_attention_decode_split_paged_bf16(
        out, pm, pl, pa, dq, dck, dcv, dpt, dseq, None, None, None, c, 0, scale,
        split_size, num_splits, batch))
    torch.cuda.synchronize()
    om, ol, oa = oracle.decode_split(q, ck, cv, pt, seq, cfg, 0, scale, split_size, num_splits)
    gm, gl, ga = pm.cpu().numpy(), pl.cpu().numpy(), pa.cpu().numpy()
    live = ~np.isnan(om)
    assert np.array_equal(live, ~np.isnan(gm)), "live split set differs"
    assert np.allclose(gm[live], om[live], rtol=1e-4, atol=1e-4)
    # l and acc are relative to each split's own maximum: compare normalised.
    assert np.allclose(gl[live], ol[live], rtol=2e-3, atol=1e-5)
    d = dim
    for i in np.nonzero(live)[0]:
        if ol[i] > 0:
            np.testing.assert_allclose(ga[i * d:(i + 1) * d] / gl[i], oa[i * d:(i + 1) * d] / ol[i],
                                       atol=2e-3, rtol=2e-3)
    gk.check(gk.flash_attention_decode_combine_bf16(out, pm, pl, pa, dseq, c, split_size,
                                                    num_splits, batch))
    torch.cuda.synchronize()
    two_phase = from_dev_bf16(out)
    one_call = _run_decode(dev, cfg, q, dck, dcv, pt, seq, 0, scale, split_size, num_splits)
    assert np.array_equal(two_phase, one_call)
    exp = oracle.decode_combine(om, ol, oa, seq, cfg, split_size, num_splits)
    assert_close(two_phase, exp, "combine of oracle partials")


@pytest.mark.parametrize("seed", range(20))
def test_decode_randomized_against_oracle(dev, seed):
    """Seeded random cases against the oracle: geometry, cache kind (ring
    with a spare page, ring of exactly the window -- full rings are split by
    ring slot --, global), page size, batch, ragged lengths including 0 and
    the window edges, planned or arbitrary split sizes, fused append or
    not, separate or in-kernel combine. Appends bit-exact, outputs within
    the north-star tolerance."""
    import torch
    rng = np.random.default_rng(4000 + seed)
    heads, dim = (8, 256) if rng.random() < 0.75 else (1, 512)
    kind = ["ring", "exact_ring", "global"][int(rng.integers(0, 3))]
    batch = int(rng.integers(1, 4))
    if kind == "global":
        page = int(rng.choice([16, 64]))
        window = 0
        seq = [int(rng.integers(0, 3000)) for _ in range(batch)]
        max_pages = (max(max(seq), 1) + 1 + page - 1) // page
    else:
        window = int(rng.choice([64, 256, 1024]))
        page = int(rng.choice([1, 4, 16]))
        edges = [0, 1, window - 1, window, window + 1, 2 * window + 5]
        seq = [int(rng.choice(edges)) if rng.random() < 0.5 else int(rng.integers(0, 3 * window))
               for _ in range(batch)]
        max_pages = window // page if kind == "exact_ring" else ring_pages(window, page)
    fused = rng.random() < 0.7
    if fused:
        seq = [n + 1 for n in seq]   # the appended token is the last live key
    cfg = cache_config(1, batch, page, max_pages, heads, dim, window)
    pt = fill_page_table(cfg, seq)
    n_rows = batch * max_pages * page
    ck0 = randn_bf16(rng, (n_rows, heads, dim))
    cv0 = randn_bf16(rng, (n_rows, heads, dim))
    q = randn_bf16(rng, (batch, 16, dim))
    scale = 1.0 / math.sqrt(dim)
    live = max(min(n, window) if window else n for n in seq)
    if rng.random() < 0.5:
        split_size, num_splits = gk.decode_split_plan(gk.make_config(*cfg), batch, max(live, 1))
    else:
        split_size = int(rng.choice([16, 20, 48, 96, 333]))
        num_splits = max(1, (live + split_size - 1) // split_size)
    exp_k, exp_v = ck0.copy(), cv0.copy()
    fused_args = None
    if fused:
        k_new = randn_bf16(rng, (batch, heads, dim))
        v_new = randn_bf16(rng, (batch, heads, dim))
        pos = [n - 1 for n in seq]
        oracle.kv_cache_write(exp_k, exp_v, cfg, pt, list(range(batch)), pos, 0, k_new, v_new)
        fused_args = (pos, k_new, v_new)
    exp = oracle.decode_attention(q, exp_k, exp_v, pt, seq, cfg, 0, scale)
    counters = None
    if fused and num_splits > 1 and rng.random() < 0.3:
        counters = torch.zeros(batch * heads, dtype=torch.int32, device=dev)
    what = (f"seed {seed}: {heads}x{dim} {kind} page {page} window {window} seq {seq} "
            f"split {split_size}x{num_splits} fused {fused} counters {counters is not None}")
    print(what, flush=True)
    ck, cv = to_dev(ck0, dev), to_dev(cv0, dev)
    got = _run_decode(dev, cfg, q, ck, cv, pt, seq, 0, scale, split_size, num_splits,
                      fused=fused_args, counters=counters)
    assert np.array_equal(from_dev_bf16(ck).reshape(exp_k.shape), exp_k), what
    assert np.array_equal(from_dev_bf16(cv).reshape(exp_v.shape), exp_v), what
    assert_close(got, exp, what)
    for b, n in enumerate(seq):
        if n == 0:
            assert not got[b].any(), what
