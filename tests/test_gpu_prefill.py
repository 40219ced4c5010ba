"""GPU parity of the chunked-prefill paged attention (MFMA kernel) against the
fp64 oracle.

The reference's prefill runs flash varlen attention over gathered K/V
(thinker_text.rs:1344-1365, attention.rs:554-664): causal masking is
bottom-right aligned (query i of n sees keys t <= i + L - n) and the
denominator has no epsilon, so the oracle runs with eps=0. Tolerance is the
bf16/f16 bar of 2e-2 (tests/_util.assert_attention_close)."""

import numpy as np
import pytest
import torch

import vpa
from oracle import oracle as orc
from tests._util import (assert_attention_close, block_tables_for, make_cache, random_words,
                         to_dev, to_host, u32)

pytestmark = pytest.mark.gpu

NAN16 = {orc.BF16: 0x7FC0, orc.F16: 0x7E00}


def prefill_case(device, code, h, kvh, d, bs, prior, qlens, seed, causal=True, nb=None,
                 mutate_bt=None, stale_nan=False, max_query_len=None, max_context_len=None,
                 pad_cols=0, scale=None):
    rng = np.random.default_rng(seed)
    prior = np.asarray(prior, dtype=np.int64)
    qlens = np.asarray(qlens, dtype=np.int64)
    lens = prior + qlens
    need = int(sum((int(L) + bs - 1) // bs for L in lens))
    nb = nb or need + 8
    kc, vc = make_cache(rng, nb, kvh, d, bs, code)
    bt = block_tables_for(rng, [max(int(L), 1) for L in lens], nb, bs, pad_cols=pad_cols)
    if stale_nan:
        # every cache slot that holds no token of any sequence is NaN
        used_k = np.zeros(kc.shape, dtype=bool)
        used_v = np.zeros(vc.shape, dtype=bool)
        for s, L in enumerate(lens):
            for t in range(int(L)):
                b, o = bt[s, t // bs], t % bs
                used_k[b, :, :, o, :] = True
                used_v[b, :, :, o] = True
        kc[~used_k] = NAN16[code]
        vc[~used_v] = NAN16[code]
    if mutate_bt is not None:
        mutate_bt(bt)
    q = random_words(rng, (int(qlens.sum()), h, d), code)
    cu = np.concatenate([[0], np.cumsum(qlens)]).astype(np.uint32)
    lens32 = lens.astype(np.uint32)
    scale = d ** -0.5 if scale is None else scale
    out = vpa.paged_attention_varlen_prefill(
        to_dev(q, code, device), to_dev(kc, code, device), to_dev(vc, code, device),
        u32(bt, device), u32(lens32, device), u32(cu, device), None, None, scale, 1.0,
        causal=causal, max_query_len=max_query_len, max_context_len=max_context_len)
    torch.cuda.synchronize()
    want = orc.prefill_attention(q, kc, vc, bt, lens32, cu, scale, causal=causal, dtype=code)
    return orc.to_f32(to_host(out), code), want


RAGGED_PRIOR = [0, 5, 31, 100, 0, 333]
RAGGED_NEW = [1, 31, 32, 33, 129, 70]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("bs", [8, 16, 32])
@pytest.mark.parametrize("code", [orc.BF16, orc.F16])
def test_prefill_qwen3_asr_shape(device, code, bs, causal):
    got, want = prefill_case(device, code, 16, 8, 128, bs, RAGGED_PRIOR, RAGGED_NEW,
                             seed=bs + 7 * code + causal, causal=causal)
    assert_attention_close(got, want, code, f"code={code} bs={bs} causal={causal}")


@pytest.mark.parametrize("d", [64, 96, 128, 192, 256])
@pytest.mark.parametrize("h,kvh", [(8, 8), (16, 8), (16, 4)])
def test_prefill_head_dims_and_groups(device, d, h, kvh):
    got, want = prefill_case(device, orc.BF16, h, kvh, d, 16, [7, 0, 260], [40, 65, 17],
                             seed=d + h + kvh)
    assert_attention_close(got, want, orc.BF16, f"d={d} h={h} kvh={kvh}")


@pytest.mark.parametrize("d,bs,code,causal", [
    (96, 32, orc.F16, True), (96, 16, orc.BF16, False), (192, 8, orc.BF16, False),
    (192, 32, orc.F16, True), (256, 8, orc.BF16, True), (256, 32, orc.BF16, False),
    (256, 16, orc.F16, True)])
def test_prefill_head_dims_block_sizes(device, d, bs, code, causal):
    """The Metal prefill's head dims (varlen_prefill.rs:15) over the block
    sizes: ragged prior and new lengths, stale NaN in every unused slot."""
    got, want = prefill_case(device, code, 16, 8, d, bs, RAGGED_PRIOR, RAGGED_NEW,
                             seed=d + bs + code + causal, causal=causal, stale_nan=True)
    assert np.isfinite(got).all()
    assert_attention_close(got, want, code, f"d={d} bs={bs} code={code} causal={causal}")


@pytest.mark.parametrize("scale", [-0.125, 1.0, 4.0])
def test_prefill_softmax_scales(device, scale):
    """Scales far from 1/sqrt(D): large ones spread a row's scores over many
    binades, so the running max moves often and the deferred rescale of O
    runs on most tiles; a negative scale flips which key dominates."""
    got, want = prefill_case(device, orc.BF16, 16, 8, 128, 16, [300, 0, 45], [90, 200, 1],
                             seed=int(scale * 8) + 40, scale=scale)
    assert_attention_close(got, want, orc.BF16, f"scale={scale}")


def test_prefill_without_prior_is_plain_causal_attention(device):
    """P = 0: the cached-causal mask reduces to the ordinary lower triangle
    (the oracle's P = 0 case is pinned to SDPA(is_causal=True) in
    tests/test_oracle.py)."""
    got, want = prefill_case(device, orc.BF16, 16, 8, 128, 16, [0], [200], seed=11)
    assert_attention_close(got, want, orc.BF16, "P=0")


def test_prefill_single_query_rows_match_decode(device):
    """n = 1 per sequence: the last position sees every key, which is exactly
    decode attention (up to decode's 1e-6 denominator term)."""
    code, h, kvh, d, bs = orc.BF16, 16, 8, 128, 16
    prior = [0, 15, 16, 17, 500, 1023]
    got, want = prefill_case(device, code, h, kvh, d, bs, prior, [1] * len(prior), seed=12)
    assert_attention_close(got, want, code, "n=1")


def test_prefill_more_queries_than_keys_gives_zero_rows(device):
    """context_lens[s] < n_s: the first n_s - L_s rows see no key (bottom-right
    alignment puts their diagonal before key 0) and are written as zeros, as
    flash attention does."""
    code, h, kvh, d, bs = orc.BF16, 8, 8, 64, 16
    rng = np.random.default_rng(13)
    nb = 16
    kc, vc = make_cache(rng, nb, kvh, d, bs, code)
    bt = np.array([[3, 4, 0, 0]], dtype=np.uint32)
    n, L = 40, 25
    q = random_words(rng, (n, h, d), code)
    cu = np.array([0, n], dtype=np.uint32)
    lens = np.array([L], dtype=np.uint32)
    out = vpa.paged_attention_varlen_prefill(
        to_dev(q, code, device), to_dev(kc, code, device), to_dev(vc, code, device),
        u32(bt, device), u32(lens, device), u32(cu, device), None, None, d ** -0.5, 1.0,
        causal=True)
    torch.cuda.synchronize()
    got = orc.to_f32(to_host(out), code)
    want = orc.prefill_attention(q, kc, vc, bt, lens, cu, d ** -0.5, causal=True, dtype=code)
    assert np.all(got[:n - L] == 0)
    assert_attention_close(got, want, code, "n > L")


def test_prefill_stale_nan_and_partial_blocks(device):
    """Unused slots of the pool (tails of last blocks, unused blocks, block 0)
    hold NaN: keys past the context are masked and their values zeroed."""
    got, want = prefill_case(device, orc.BF16, 16, 8, 128, 16, [3, 44, 0], [20, 37, 9],
                             seed=14, stale_nan=True)
    assert_attention_close(got, want, orc.BF16, "stale NaN")


def test_prefill_invalid_block_ids_are_skipped(device):
    def mutate(bt):
        bt[0, 1] = 1 << 30     # out of the pool: its tokens are absent
        bt[1, 0] = 0xFFFFFFFF
    got, want = prefill_case(device, orc.BF16, 16, 8, 128, 16, [40, 20], [30, 50], seed=15,
                             mutate_bt=mutate)
    assert_attention_close(got, want, orc.BF16, "invalid blocks")


@pytest.mark.parametrize("col", [2, 4, 7])
def test_prefill_absent_block_in_either_tile_of_a_step(device, col):
    """The kernel consumes keys in steps of two 32-key tiles. An absent block
    (id past the pool) in the second tile of step 0 (column 2), the first
    tile of step 1 (column 4) or the second tile of step 1 (column 7), over a
    pool whose unused slots hold NaN (block 0, read in place of the absent
    block, among them), must be masked and its values zeroed in whichever
    tile it falls."""
    def mutate(bt):
        bt[0, col] = 1 << 30
    got, want = prefill_case(device, orc.BF16, 16, 8, 128, 16, [100, 60], [40, 50],
                             seed=16 + col, stale_nan=True, mutate_bt=mutate)
    assert np.isfinite(got).all()
    assert_attention_close(got, want, orc.BF16, f"absent column {col}")


@pytest.mark.parametrize("col", [9, 13])
def test_prefill_absent_block_in_a_later_step(device, col):
    """Steps 2 and later take their block ids from the window loaded two
    steps ahead and learn only whether every block is in the pool; a step
    with an absent block (column 9: step 2, column 13: step 3) works its
    mask out from its ids loaded again."""
    def mutate(bt):
        bt[0, col] = 1 << 30
    got, want = prefill_case(device, orc.BF16, 16, 8, 128, 16, [200, 60], [40, 50],
                             seed=20 + col, stale_nan=True, mutate_bt=mutate)
    assert np.isfinite(got).all()
    assert_attention_close(got, want, orc.BF16, f"absent column {col}")


def test_prefill_padded_table_columns_and_frozen_maxima(device):
    """Extra zero columns in block_tables and host maxima above the true ones
    (a grid sized for a larger batch) change nothing."""
    got, want = prefill_case(device, orc.BF16, 16, 8, 128, 16, [10, 90], [50, 7], seed=16,
                             pad_cols=60, max_query_len=300, max_context_len=900)
    assert_attention_close(got, want, orc.BF16, "padded")


def test_prefill_max_query_len_clamps_rows(device):
    """Rows past max_query_len are not computed (their output is untouched)."""
    code, h, kvh, d, bs = orc.BF16, 16, 8, 128, 16
    rng = np.random.default_rng(17)
    prior, qlens = [8, 0], [50, 20]
    lens = np.array(prior) + np.array(qlens)
    nb = 16
    kc, vc = make_cache(rng, nb, kvh, d, bs, code)
    bt = block_tables_for(rng, lens, nb, bs)
    q = random_words(rng, (70, h, d), code)
    cu = np.array([0, 50, 70], dtype=np.uint32)
    out = torch.full((70, h, d), 7.0, dtype=torch.bfloat16, device=device)
    vpa.paged_attention_varlen_prefill(
        to_dev(q, code, device), to_dev(kc, code, device), to_dev(vc, code, device),
        u32(bt, device), u32(lens.astype(np.uint32), device), u32(cu, device), None, None,
        d ** -0.5, 1.0, causal=True, max_query_len=32, max_context_len=int(lens.max()),
        out=out)
    torch.cuda.synchronize()
    got = orc.to_f32(to_host(out), code)
    # with n clamped to 32 and L unchanged the shift L - n grows; the oracle
    # sees the same clamped problem
    cu_c = np.array([0, 32], dtype=np.uint32)
    want0 = orc.prefill_attention(q[:32], kc, vc, bt[:1], lens[:1].astype(np.uint32), cu_c,
                                  d ** -0.5, causal=True, dtype=code)
    assert_attention_close(got[:32], want0, code, "clamped seq 0")
    assert np.all(got[32:50] == 7.0)
    want1 = orc.prefill_attention(q[50:], kc, vc, bt[1:], lens[1:].astype(np.uint32),
                                  np.array([0, 20], dtype=np.uint32), d ** -0.5, causal=True,
                                  dtype=code)
    assert_attention_close(got[50:], want1, code, "seq 1")


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("code", [orc.BF16, orc.F16])
def test_prefill_long_context(device, code, causal):
    """A 16 000-token prior (1000 blocks; the last query tile walks ~250
    two-tile steps) beside a short sequence: the block-id windows near the
    table's end, the lazy rescale and the tail masks over a long run."""
    got, want = prefill_case(device, code, 16, 8, 128, 16, [16000, 40], [160, 24], seed=31,
                             causal=causal)
    assert_attention_close(got, want, code, "long context")


def test_prefill_long_context_large_scale(device):
    """Logits ten times larger than the usual scale give (log2) spreads far
    beyond the rescale slack: the reference max moves many times along a
    12 000-token context."""
    got, want = prefill_case(device, orc.BF16, 16, 8, 128, 16, [12000], [96], seed=32,
                             scale=10 * 128 ** -0.5)
    assert_attention_close(got, want, orc.BF16, "long context, scale 10/sqrt(d)")


def test_prefill_config_c4(device):
    """c4 end to end on the GPU: append the 512 new tokens of each of the 64
    sequences with reshape_and_cache, then prefill; every sequence and head
    of the call is checked against the oracle (all 64 share the pool)."""
    from vpa import workloads
    w = workloads.c4()
    code = orc.BF16
    rng = np.random.default_rng(w.seed)
    h, kvh, d, bs = w.num_heads, w.num_kv_heads, w.head_dim, w.block_size
    kc, vc = make_cache(rng, w.num_blocks, kvh, d, bs, code)
    tq = int(w.query_lens.sum())
    q = random_words(rng, (tq, h, d), code)
    knew = random_words(rng, (tq, kvh, d), code)
    vnew = random_words(rng, (tq, kvh, d), code)
    slots = w.slot_mapping()
    kc_d, vc_d = to_dev(kc, code, device), to_dev(vc, code, device)
    vpa.reshape_and_cache(to_dev(knew, code, device), to_dev(vnew, code, device), None, None,
                          kc_d, vc_d, torch.from_numpy(slots).to(device))
    cu = w.cu_seqlens_q
    lens = w.context_lens
    out = vpa.paged_attention_varlen_prefill(
        to_dev(q, code, device), kc_d, vc_d, u32(w.block_tables, device), u32(lens, device),
        u32(cu, device), None, None, d ** -0.5, 1.0, causal=True,
        max_query_len=int(w.query_lens.max()), max_context_len=int(lens.max()))
    torch.cuda.synchronize()
    got = orc.to_f32(to_host(out), code)
    kc_h, vc_h = to_host(kc_d), to_host(vc_d)
    want = orc.prefill_attention(q, kc_h, vc_h, w.block_tables, lens, cu, d ** -0.5, causal=True,
                                 dtype=code)
    for s in range(len(lens)):
        rows = slice(int(cu[s]), int(cu[s + 1]))
        assert_attention_close(got[rows], want[rows], code, f"c4 seq {s}")


def test_prefill_matches_gather_then_dense_attention(device):
    """The reference's two-pass form: gather_kv_cache to packed K/V, then
    causal attention over it (computed here on the CPU in float64 with the
    bottom-right mask) agrees with the fused kernel."""
    code, h, kvh, d, bs = orc.BF16, 16, 8, 128, 16
    rng = np.random.default_rng(18)
    prior, qlens = [30, 0, 77], [18, 40, 5]
    lens = (np.array(prior) + np.array(qlens)).astype(np.uint32)
    nb = 40
    kc, vc = make_cache(rng, nb, kvh, d, bs, code)
    bt = block_tables_for(rng, lens, nb, bs)
    q = random_words(rng, (int(sum(qlens)), h, d), code)
    cu_q = np.concatenate([[0], np.cumsum(qlens)]).astype(np.uint32)
    cu_kv = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32)
    kc_d, vc_d = to_dev(kc, code, device), to_dev(vc, code, device)
    out = vpa.paged_attention_varlen_prefill(
        to_dev(q, code, device), kc_d, vc_d, u32(bt, device), u32(lens, device),
        u32(cu_q, device), None, None, d ** -0.5, 1.0, causal=True)
    gk, gv = vpa.gather_kv_cache(kc_d, vc_d, None, None, u32(bt, device), u32(cu_kv, device),
                                 torch.bfloat16)
    torch.cuda.synchronize()
    got = torch.from_numpy(orc.to_f32(to_host(out), code)).double()
    gk = gk.float().cpu().double()
    gv = gv.float().cpu().double()
    qd = torch.from_numpy(orc.to_f32(q, code)).double()
    for s in range(3):
        n, L = qlens[s], int(lens[s])
        Q = qd[cu_q[s]:cu_q[s + 1]].transpose(0, 1)                      # [H, n, D]
        K = gk[cu_kv[s]:cu_kv[s + 1]].transpose(0, 1).repeat_interleave(2, 0)
        V = gv[cu_kv[s]:cu_kv[s + 1]].transpose(0, 1).repeat_interleave(2, 0)
        mask = torch.from_numpy(np.tril(np.ones((n, L), dtype=bool), k=L - n))
        want = torch.nn.functional.scaled_dot_product_attention(Q, K, V, attn_mask=mask,
                                                                scale=d ** -0.5)
        g = got[cu_q[s]:cu_q[s + 1]].transpose(0, 1)
        assert_attention_close(g.numpy(), want.numpy(), code, f"two-pass seq {s}")


@pytest.mark.parametrize("eps", [1e-6, 0.5, 3.0])
@pytest.mark.parametrize("causal", [False, True])
def test_prefill_denominator_epsilon(device, eps, causal):
    """denom_eps is added to the softmax denominator relative to the row's
    true max (1e-6 is the Metal kernel's, prefill_paged_attn.metal:1300).
    Large values move the output far beyond the tolerance, so a missing or
    mis-scaled epsilon fails; a large softmax scale makes the kernel's
    reference max trail the true max so the rescaling of the epsilon is
    exercised."""
    rng = np.random.default_rng(int(eps * 100) + causal)
    code, h, kvh, d, bs = orc.BF16, 16, 8, 128, 16
    prior, qlens = np.array([40, 0, 300]), np.array([70, 33, 129])
    lens = prior + qlens
    nb = int(((lens + bs - 1) // bs).sum()) + 8
    kc, vc = make_cache(rng, nb, kvh, d, bs, code)
    bt = block_tables_for(rng, lens, nb, bs)
    q = random_words(rng, (int(qlens.sum()), h, d), code)
    cu = np.concatenate([[0], np.cumsum(qlens)]).astype(np.uint32)
    for scale in (d ** -0.5, 2.0):
        out = vpa.paged_attention_varlen_prefill(
            to_dev(q, code, device), to_dev(kc, code, device), to_dev(vc, code, device),
            u32(bt, device), u32(lens, device), u32(cu, device), None, None, scale, 1.0,
            causal=causal, denom_eps=eps)
        torch.cuda.synchronize()
        want = orc.prefill_attention(q, kc, vc, bt, lens.astype(np.uint32), cu, scale,
                                     causal=causal, dtype=code, eps=eps)
        assert_attention_close(orc.to_f32(to_host(out), code), want, code,
                               f"eps={eps} causal={causal} scale={scale}")
    if eps >= 0.5:  # the epsilon matters at this size: eps = 0 is far off
        none = orc.prefill_attention(q, kc, vc, bt, lens.astype(np.uint32), cu, scale,
                                     causal=causal, dtype=code, eps=0.0)
        err = np.abs(orc.to_f32(to_host(out), code) - none).max() / np.abs(none).max()
        assert err > 0.05
