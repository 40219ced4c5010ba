"""Pins of the CPU oracle (oracle/vpa_oracle.c) — CPU only.

Each check is chosen so that a plausible slip in the oracle (a transposed
tile, a wrong GQA map, a missing 1e-6, a shifted causal diagonal) fails it,
and none retypes the oracle's own formula:

* cache layout: the reference's host-side inverse of the layout
  (``vasr-models/src/model/generation.rs:338-440``: transpose(0,1),
  transpose(2,3), reshape) applied with numpy transposes;
* reshape_and_cache: PAD_SLOT_ID skip (``paged_kv_cache.rs:697-700``),
  canary bytes outside the target slots, bit patterns (NaN payloads)
  preserved;
* gather_kv_cache: append -> gather round trip;
* decode and prefill attention: torch's scaled_dot_product_attention (a
  library routine) on the gathered K/V with repeat_interleave GQA, and the
  1e-6 term pinned through torch.logsumexp; closed forms (L=1, constant keys,
  one-hot values revealing the causal mask of ``attention.rs:78-149``, KAT
  ``attention.rs:870-909``); the reference's packed-vs-unpacked test inputs
  (``attention.rs:949-1041``, q=i*0.01, kv=i*0.02+1, tolerance 1e-4);
  physical-block permutation invariance.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.filterwarnings("ignore::UserWarning")


def make_cache(nb, kvh, d, bs, code, rng, fill=None):
    x = 16 // (4 if code == orc.F32 else 2)
    kshape = (nb, kvh, d // x, bs, x)
    vshape = (nb, kvh, d, bs)
    if fill is None:
        k = orc.from_f32(rng.standard_normal(kshape).astype(np.float32), code)
        v = orc.from_f32(rng.standard_normal(vshape).astype(np.float32), code)
    else:
        dt = np.float32 if code == orc.F32 else np.uint16
        k = np.full(kshape, fill, dtype=dt)
        v = np.full(vshape, fill, dtype=dt)
    return np.ascontiguousarray(k), np.ascontiguousarray(v)


def inverse_layout(key_cache, value_cache, table, length):
    """Host inverse of the paged layout as the reference writes it
    (generation.rs:338-440): per sequence, cat the blocks of its table, then
    K: transpose(0,1).transpose(2,3).reshape(KVH, NB*BS, D)[:, :len];
    V: the same on [NB, KVH, D, BS]."""
    kb = key_cache[np.asarray(table)]            # [nb, KVH, D/x, BS, x]
    vb = value_cache[np.asarray(table)]          # [nb, KVH, D, BS]
    nbk, kvh, dx, bs, x = kb.shape
    k = kb.transpose(1, 0, 2, 3, 4).transpose(0, 1, 3, 2, 4).reshape(kvh, nbk * bs, dx * x)
    v = vb.transpose(1, 0, 2, 3).transpose(0, 1, 3, 2).reshape(kvh, nbk * bs, dx * x)
    return k[:, :length], v[:, :length]


@pytest.mark.parametrize("code", [orc.F32, orc.BF16, orc.F16])
@pytest.mark.parametrize("bs", [8, 16, 32])
def test_reshape_and_cache_matches_reference_inverse(code, bs):
    rng = np.random.default_rng(10 + bs + code)
    kvh, d, nb = 2, 64, 24
    length = 3 * bs + 5
    table = rng.permutation(nb)[: (length + bs - 1) // bs]
    kc, vc = make_cache(nb, kvh, d, bs, code, rng, fill=0)
    k = orc.from_f32(rng.standard_normal((length, kvh, d)).astype(np.float32), code)
    v = orc.from_f32(rng.standard_normal((length, kvh, d)).astype(np.float32), code)
    pos = np.arange(length)
    slots = table[pos // bs].astype(np.int64) * bs + pos % bs
    orc.reshape_and_cache(k, v, kc, vc, slots, dtype=code)
    ki, vi = inverse_layout(kc, vc, table, length)
    np.testing.assert_array_equal(ki, k.transpose(1, 0, 2))
    np.testing.assert_array_equal(vi, v.transpose(1, 0, 2))


def test_reshape_and_cache_pad_slots_and_canary():
    rng = np.random.default_rng(7)
    kvh, d, bs, nb = 2, 64, 16, 8
    kc, vc = make_cache(nb, kvh, d, bs, orc.BF16, rng, fill=0xABCD)
    k0, v0 = kc.copy(), vc.copy()
    # random words including NaN/Inf bit patterns: the copy must keep them
    k = rng.integers(0, 1 << 16, size=(6, kvh, d), dtype=np.uint16)
    v = rng.integers(0, 1 << 16, size=(6, kvh, d), dtype=np.uint16)
    k[0, 0, :4] = [0x7FC1, 0xFF80, 0x7F80, 0x0001]
    slots = np.array([5, -1, 17, nb * bs, 127, -7], dtype=np.int64)  # -1/-7 pad, nb*bs out of range
    orc.reshape_and_cache(k, v, kc, vc, slots, dtype=orc.BF16)
    x = 8
    touched_k = np.zeros(kc.shape, dtype=bool)
    touched_v = np.zeros(vc.shape, dtype=bool)
    for t, s in enumerate(slots):
        if s < 0 or s >= nb * bs:
            continue
        blk, off = divmod(int(s), bs)
        for j in range(kvh):
            for dd in range(d):
                assert kc[blk, j, dd // x, off, dd % x] == k[t, j, dd]
                assert vc[blk, j, dd, off] == v[t, j, dd]
                touched_k[blk, j, dd // x, off, dd % x] = True
                touched_v[blk, j, dd, off] = True
    assert touched_k.sum() == 3 * kvh * d
    np.testing.assert_array_equal(kc[~touched_k], k0[~touched_k])
    np.testing.assert_array_equal(vc[~touched_v], v0[~touched_v])


@pytest.mark.parametrize("code", [orc.F32, orc.BF16])
def test_gather_round_trip(code):
    rng = np.random.default_rng(3)
    kvh, d, bs, nb = 2, 64, 16, 40
    lens = np.array([37, 1, 16, 50])
    kc, vc = make_cache(nb, kvh, d, bs, code, rng)
    perm = rng.permutation(np.arange(1, nb))
    cols = int(max((lens + bs - 1) // bs))
    bt = np.zeros((len(lens), cols), dtype=np.uint32)
    rows_k, rows_v, slots = [], [], []
    off = 0
    for s, L in enumerate(lens):
        n = (L + bs - 1) // bs
        bt[s, :n] = perm[off:off + n]
        off += n
        pos = np.arange(L)
        slots.append(bt[s, pos // bs].astype(np.int64) * bs + pos % bs)
        rows_k.append(orc.from_f32(rng.standard_normal((L, kvh, d)).astype(np.float32), code))
        rows_v.append(orc.from_f32(rng.standard_normal((L, kvh, d)).astype(np.float32), code))
    k = np.ascontiguousarray(np.concatenate(rows_k))
    v = np.ascontiguousarray(np.concatenate(rows_v))
    orc.reshape_and_cache(k, v, kc, vc, np.concatenate(slots), dtype=code)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32)
    gk, gv = orc.gather_kv_cache(kc, vc, bt, cu, dtype=code)
    np.testing.assert_array_equal(gk, k)
    np.testing.assert_array_equal(gv, v)


def _random_decode(rng, code, b, h, kvh, d, bs, lens, nb):
    kc, vc = make_cache(nb, kvh, d, bs, code, rng)
    cols = int(max((np.asarray(lens) + bs - 1) // bs))
    bt = np.zeros((b, cols), dtype=np.uint32)
    for s, L in enumerate(lens):
        n = (L + bs - 1) // bs
        bt[s, :n] = rng.choice(nb, size=n, replace=False)
    q = orc.from_f32(rng.standard_normal((b, h, d)).astype(np.float32), code)
    return q, kc, vc, bt


def _sdpa_decode(q, kc, vc, bt, lens, scale, code):
    """torch SDPA (float64, CPU) on K/V recovered with the reference inverse."""
    b, h, d = q.shape
    kvh = kc.shape[1]
    outs, lse = [], []
    for s, L in enumerate(lens):
        n = (L + kc.shape[3] - 1) // kc.shape[3]
        ki, vi = inverse_layout(kc, vc, bt[s, :n], L)
        K = torch.from_numpy(orc.to_f32(ki, code).astype(np.float64))
        V = torch.from_numpy(orc.to_f32(vi, code).astype(np.float64))
        K = K.repeat_interleave(h // kvh, dim=0)
        V = V.repeat_interleave(h // kvh, dim=0)
        Q = torch.from_numpy(orc.to_f32(q[s], code).astype(np.float64))[:, None, :]
        o = torch.nn.functional.scaled_dot_product_attention(Q, K, V, scale=scale)[:, 0, :]
        logits = (Q @ K.transpose(1, 2))[:, 0, :] * scale
        m = logits.max(dim=1, keepdim=True).values
        S = torch.exp(torch.logsumexp(logits, dim=1, keepdim=True) - m)  # sum exp(s - max)
        outs.append(o)
        lse.append(S)
    return torch.stack(outs).numpy(), torch.stack(lse).numpy()


@pytest.mark.parametrize("code,h,kvh,bs", [(orc.F32, 16, 8, 16), (orc.BF16, 16, 8, 16),
                                           (orc.F16, 8, 2, 8), (orc.F32, 4, 4, 32)])
def test_decode_oracle_matches_torch_sdpa(code, h, kvh, bs):
    rng = np.random.default_rng(100 + h + bs)
    d, nb = 128, 96
    lens = [1, 17, 200, 333]
    q, kc, vc, bt = _random_decode(rng, code, len(lens), h, kvh, d, bs, lens, nb)
    scale = d ** -0.5
    got = orc.paged_attention(q, kc, vc, bt, np.array(lens), max(lens), scale, dtype=code)
    want, S = _sdpa_decode(q, kc, vc, bt, lens, scale, code)
    # the oracle divides by (S + 1e-6); SDPA by S
    np.testing.assert_allclose(got * (S + 1e-6) / S, want, rtol=1e-10, atol=1e-12)


def test_decode_closed_forms():
    rng = np.random.default_rng(5)
    code, h, kvh, d, bs, nb = orc.F32, 4, 2, 64, 16, 16
    # L = 1: out = V[t0] / (1 + 1e-6)
    q, kc, vc, bt = _random_decode(rng, code, 1, h, kvh, d, bs, [1], nb)
    out = orc.paged_attention(q, kc, vc, bt, np.array([1]), 1, 0.1, dtype=code)
    for hh in range(h):
        v0 = vc[bt[0, 0], hh // 2, :, 0].astype(np.float64)
        np.testing.assert_allclose(out[0, hh], v0 / (1 + 1e-6), rtol=1e-12)
    # constant keys: uniform weights -> mean of V * L/(L+1e-6)
    L = 40
    q, kc, vc, bt = _random_decode(rng, code, 1, h, kvh, d, bs, [L], nb)
    kc[:] = 0.25
    out = orc.paged_attention(q, kc, vc, bt, np.array([L]), L, 0.3, dtype=code)
    _, vi = inverse_layout(kc, vc, bt[0, :3], L)
    for hh in range(h):
        np.testing.assert_allclose(out[0, hh], vi[hh // 2].astype(np.float64).mean(0) * L / (L + 1e-6),
                                   rtol=1e-10)


def test_decode_permutation_invariance_and_invalid_blocks():
    rng = np.random.default_rng(9)
    code, h, kvh, d, bs, nb = orc.BF16, 16, 8, 128, 16, 32
    L = 70
    q, kc, vc, bt = _random_decode(rng, code, 1, h, kvh, d, bs, [L], nb)
    base = orc.paged_attention(q, kc, vc, bt, np.array([L]), L, 0.088, dtype=code)
    perm = rng.permutation(nb)
    kc2, vc2 = np.empty_like(kc), np.empty_like(vc)
    kc2[perm] = kc
    vc2[perm] = vc
    bt2 = perm[bt].astype(np.uint32)
    moved = orc.paged_attention(q, kc2, vc2, bt2, np.array([L]), L, 0.088, dtype=code)
    np.testing.assert_allclose(moved, base, rtol=1e-12, atol=1e-15)
    # a block id >= num_blocks drops that block's tokens: same as attending to
    # the remaining tokens only (here: tokens 16..69 after moving block 0 out)
    bt3 = bt.copy()
    bt3[0, 0] = nb + 5
    part = orc.paged_attention(q, kc, vc, bt3, np.array([L]), L, 0.088, dtype=code)
    ki, vi = inverse_layout(kc, vc, bt[0, :5], L)
    Q = orc.to_f32(q[0], code).astype(np.float64)
    K = orc.to_f32(ki, code).astype(np.float64)[:, 16:]
    V = orc.to_f32(vi, code).astype(np.float64)[:, 16:]
    for hh in range(h):
        lg = K[hh // 2] @ Q[hh] * 0.088
        p = np.exp(lg - lg.max())
        np.testing.assert_allclose(part[0, hh], p @ V[hh // 2] / (p.sum() + 1e-6), rtol=1e-10)


def _prefill_case(rng, code, h, kvh, d, bs, prior, qlens, nb):
    lens = np.asarray(prior) + np.asarray(qlens)
    kc, vc = make_cache(nb, kvh, d, bs, code, rng)
    cols = int(max((lens + bs - 1) // bs))
    bt = np.zeros((len(lens), cols), dtype=np.uint32)
    ids = rng.permutation(nb)
    off = 0
    for s, L in enumerate(lens):
        n = (L + bs - 1) // bs
        bt[s, :n] = ids[off:off + n]
        off += n
    tq = int(sum(qlens))
    q = orc.from_f32(rng.standard_normal((tq, h, d)).astype(np.float32), code)
    cu = np.concatenate([[0], np.cumsum(qlens)]).astype(np.uint32)
    return q, kc, vc, bt, lens.astype(np.uint32), cu


@pytest.mark.parametrize("causal", [True, False])
def test_prefill_oracle_matches_torch_sdpa_with_cached_mask(causal):
    rng = np.random.default_rng(21)
    code, h, kvh, d, bs, nb = orc.BF16, 8, 4, 64, 16, 64
    prior, qlens = [0, 19, 40], [23, 9, 1]
    q, kc, vc, bt, lens, cu = _prefill_case(rng, code, h, kvh, d, bs, prior, qlens, nb)
    scale = d ** -0.5
    got = orc.prefill_attention(q, kc, vc, bt, lens, cu, scale, causal=causal, dtype=code)
    got_eps = orc.prefill_attention(q, kc, vc, bt, lens, cu, scale, causal=causal, dtype=code,
                                    eps=1e-6)
    assert not np.array_equal(got, got_eps)
    for s in range(len(lens)):
        L, n, P = int(lens[s]), qlens[s], prior[s]
        ki, vi = inverse_layout(kc, vc, bt[s, :(L + bs - 1) // bs], L)
        K = torch.from_numpy(orc.to_f32(ki, code).astype(np.float64)).repeat_interleave(2, 0)
        V = torch.from_numpy(orc.to_f32(vi, code).astype(np.float64)).repeat_interleave(2, 0)
        Q = torch.from_numpy(orc.to_f32(q[cu[s]:cu[s + 1]], code).astype(np.float64)).transpose(0, 1)
        if causal:
            # make_causal_mask_cached: key kv allowed for query i iff kv <= P + i
            mask = torch.from_numpy(np.tril(np.ones((n, L), dtype=bool), k=P))
        else:
            mask = torch.ones((n, L), dtype=torch.bool)
        want = torch.nn.functional.scaled_dot_product_attention(Q, K, V, attn_mask=mask, scale=scale)
        logits = (Q @ K.transpose(1, 2)) * scale
        logits = logits.masked_fill(~mask, float("-inf"))
        m = logits.max(dim=-1, keepdim=True).values
        S = torch.exp(torch.logsumexp(logits, dim=-1, keepdim=True) - m)
        g = torch.from_numpy(got[cu[s]:cu[s + 1]]).transpose(0, 1)
        torch.testing.assert_close(g, want, rtol=1e-10, atol=1e-12)
        # the Metal kernel's epsilon variant divides by S + 1e-6
        ge = torch.from_numpy(got_eps[cu[s]:cu[s + 1]]).transpose(0, 1)
        torch.testing.assert_close(ge * (S + 1e-6) / S, want, rtol=1e-10, atol=1e-12)
    if prior[0] == 0 and causal:
        # P = 0 reduces to plain causal attention
        L = qlens[0]
        ki, vi = inverse_layout(kc, vc, bt[0, :(L + bs - 1) // bs], L)
        K = torch.from_numpy(orc.to_f32(ki, code).astype(np.float64)).repeat_interleave(2, 0)
        V = torch.from_numpy(orc.to_f32(vi, code).astype(np.float64)).repeat_interleave(2, 0)
        Q = torch.from_numpy(orc.to_f32(q[:L], code).astype(np.float64)).transpose(0, 1)
        want = torch.nn.functional.scaled_dot_product_attention(Q, K, V, is_causal=True, scale=scale)
        g = torch.from_numpy(got[:L]).transpose(0, 1)
        torch.testing.assert_close(g, want, rtol=2e-6, atol=1e-9)


def test_prefill_cached_causal_mask_kat():
    """attention.rs:870-909: cache_len=3, new_len=2 -> query 0 (abs 3) sees
    keys 0..3, query 1 (abs 4) sees all 5. Keys are zero so visible keys get
    equal weight; one-hot values reveal which keys were seen."""
    code, h, kvh, d, bs = orc.F32, 1, 1, 64, 8
    nb = 2
    kc = np.zeros((nb, kvh, d // 4, bs, 4), dtype=np.float32)
    vc = np.zeros((nb, kvh, d, bs), dtype=np.float32)
    for t in range(5):
        vc[1, 0, t, t] = 1.0          # token t lives in block 1 offset t; V_t = e_t
    bt = np.array([[1]], dtype=np.uint32)
    q = np.ones((2, h, d), dtype=np.float32)
    out = orc.prefill_attention(q, kc, vc, bt, np.array([5], dtype=np.uint32),
                                np.array([0, 2], dtype=np.uint32), 1.0, causal=True, dtype=code)
    np.testing.assert_allclose(out[0, 0, :5], np.array([1, 1, 1, 1, 0]) / 4, rtol=1e-12)
    np.testing.assert_allclose(out[1, 0, :5], np.ones(5) / 5, rtol=1e-12)


def test_prefill_matches_reference_packed_vs_unpacked_kat():
    """attention.rs:949-1041: batch 2, seq 4, head_dim 32, 2 q heads / 1 kv
    head, query_lens = kv_lens = [3, 2], q = i*0.01, kv = i*0.02 + 1 (K = V),
    causal, checked against per-sequence matmul/softmax/matmul at 1e-4."""
    d, h, kvh, bs = 32, 2, 1, 4
    qfull = (np.arange(2 * h * 4 * d, dtype=np.float32) * 0.01).reshape(2, h, 4, d)
    qlens = [3, 2]
    packed = (np.arange(5 * kvh * d, dtype=np.float32) * 0.02 + 1.0).reshape(5, kvh, d)
    nb = 4
    kc = np.zeros((nb, kvh, d // 4, bs, 4), dtype=np.float32)
    vc = np.zeros((nb, kvh, d, bs), dtype=np.float32)
    bt = np.array([[2], [3]], dtype=np.uint32)
    slots = np.array([8, 9, 10, 12, 13], dtype=np.int64)
    orc.reshape_and_cache(packed, packed.copy(), kc, vc, slots, dtype=orc.F32)
    q = np.ascontiguousarray(np.concatenate([qfull[0, :, :3].transpose(1, 0, 2),
                                             qfull[1, :, :2].transpose(1, 0, 2)]))
    out = orc.prefill_attention(q, kc, vc, bt, np.array([3, 2], dtype=np.uint32),
                                np.array([0, 3, 5], dtype=np.uint32), d ** -0.5, causal=True,
                                dtype=orc.F32)
    start = 0
    for s, n in enumerate(qlens):
        kv = torch.from_numpy(packed[start:start + n].transpose(1, 0, 2)).repeat_interleave(2, 0)
        qr = torch.from_numpy(qfull[s, :, :n])
        w = qr @ kv.transpose(1, 2) * d ** -0.5
        w = w + torch.triu(torch.full((n, n), float("-inf")), 1)
        ref = torch.softmax(w, dim=-1) @ kv
        got = torch.from_numpy(out[start:start + n]).transpose(0, 1).float()
        assert (got - ref).abs().max().item() <= 1e-4
        start += n


def test_cpu_baseline_matches_oracle():
    rng = np.random.default_rng(11)
    code, h, kvh, d, bs, nb = orc.BF16, 16, 8, 128, 16, 64
    lens = np.array([100, 5, 260], dtype=np.uint32)
    q, kc, vc, bt = _random_decode(rng, code, 3, h, kvh, d, bs, lens, nb)
    nk = orc.from_f32(rng.standard_normal((3, kvh, d)).astype(np.float32), code)
    nv = orc.from_f32(rng.standard_normal((3, kvh, d)).astype(np.float32), code)
    pos = lens.astype(np.int64) - 1
    slots = bt[np.arange(3), pos // bs].astype(np.int64) * bs + pos % bs
    kc2, vc2 = kc.copy(), vc.copy()
    out, threads = orc.cpu_baseline_decode_step(q, nk, nv, slots, kc2, vc2, bt, lens, d ** -0.5,
                                                dtype=code)
    assert threads >= 1
    orc.reshape_and_cache(nk, nv, kc, vc, slots, dtype=code)
    np.testing.assert_array_equal(kc, kc2)
    want = orc.paged_attention(q, kc, vc, bt, lens, int(lens.max()), d ** -0.5, dtype=code)
    np.testing.assert_allclose(out, want, rtol=1e-4, atol=1e-5)


# ---- fp8 (E4M3FN) cache ------------------------------------------------------

def test_fp8_decode_of_every_byte_matches_torch():
    """All 256 E4M3FN codes against torch.float8_e4m3fn, plus the format's
    closed forms (bias 7, subnormals m * 2^-9, S.1111.111 = NaN)."""
    codes = np.arange(256, dtype=np.uint8)
    got = orc.fp8_to_f32(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(got[~np.isnan(got)], ref[~np.isnan(ref)])
    assert got[0x7E] == 448.0 and got[0x38] == 1.0 and got[0x08] == 2.0 ** -6
    assert got[0x01] == 2.0 ** -9 and np.isnan(got[0x7F]) and np.isnan(got[0xFF])
    assert got[0x80] == 0.0 and np.signbit(got[0x80])


def test_fp8_encode_matches_torch_in_range():
    """Round to nearest even for every bf16 bit pattern below 448, exact
    midpoints between neighbouring codes (ties), and random values."""
    x = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    fin = orc.fp8_to_f32(np.arange(256, dtype=np.uint8))
    pos = np.sort(np.unique(fin[np.isfinite(fin) & (fin >= 0)]))
    mids = ((pos[:-1].astype(np.float64) + pos[1:]) / 2).astype(np.float32)
    rng = np.random.default_rng(7)
    x = np.concatenate([x, mids, -mids, rng.standard_normal(1 << 20).astype(np.float32) * 40,
                        rng.random(1 << 18).astype(np.float32) * np.float32(0.03)])
    x = x[np.isfinite(x) & (np.abs(x) < 448)]
    got = orc.fp8_from_f32(x)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(got, ref)
    # ties went to the even code (e.g. 1.0625 is halfway between 1.0 and 1.125)
    assert orc.fp8_from_f32(np.float32([1.0625, 1.1875]))[0] == 0x38
    assert orc.fp8_from_f32(np.float32([1.1875]))[0] == 0x3A


def test_fp8_encode_saturates_and_keeps_nan():
    x = np.float32([448.0, 449.0, 464.0, 480.0, 1e6, np.inf, -448.0, -500.0, -np.inf, np.nan])
    got = orc.fp8_from_f32(x)
    np.testing.assert_array_equal(got[:6], [0x7E] * 6)
    np.testing.assert_array_equal(got[6:9], [0xFE] * 3)
    assert got[9] & 0x7F == 0x7F


def test_fp8_encode_decode_idempotent():
    codes = np.arange(256, dtype=np.uint8)
    vals = orc.fp8_to_f32(codes)
    fin = np.isfinite(vals)
    np.testing.assert_array_equal(orc.fp8_from_f32(vals[fin]), codes[fin])


@pytest.mark.parametrize("code", [orc.BF16, orc.F32])
def test_fp8_append_gather_round_trip(code):
    """append into an fp8 cache then gather: each value comes back as
    fp8(x / scale) * scale in the output type; the cache bytes sit where the
    reference's layout inverse (x = 16) puts them."""
    rng = np.random.default_rng(31 + code)
    kvh, d, bs, nb = 2, 64, 16, 24
    length = 3 * bs + 7
    table = rng.permutation(nb)[: (length + bs - 1) // bs]
    kc = np.zeros((nb, kvh, d // 16, bs, 16), dtype=np.uint8)
    vc = np.zeros((nb, kvh, d, bs), dtype=np.uint8)
    k = orc.from_f32((rng.standard_normal((length, kvh, d)) * 30).astype(np.float32), code)
    v = orc.from_f32((rng.standard_normal((length, kvh, d)) * 30).astype(np.float32), code)
    pos = np.arange(length)
    slots = table[pos // bs].astype(np.int64) * bs + pos % bs
    ks, vs = 0.5, 2.0
    orc.reshape_and_cache_fp8(k, v, kc, vc, slots, code, ks, vs)
    ki, vi = inverse_layout(kc, vc, table, length)
    kf = orc.to_f32(k, code) if code != orc.F32 else k
    vf = orc.to_f32(v, code) if code != orc.F32 else v
    np.testing.assert_array_equal(ki, orc.fp8_from_f32(kf / np.float32(ks)).transpose(1, 0, 2))
    np.testing.assert_array_equal(vi, orc.fp8_from_f32(vf / np.float32(vs)).transpose(1, 0, 2))
    cu = np.array([0, length], dtype=np.uint32)
    gk, gv = orc.gather_kv_cache_fp8(kc, vc, table[None, :].astype(np.uint32), cu, orc.F32, ks, vs)
    np.testing.assert_array_equal(gk, orc.fp8_to_f32(ki.transpose(1, 0, 2)) * np.float32(ks))
    np.testing.assert_array_equal(gv, orc.fp8_to_f32(vi.transpose(1, 0, 2)) * np.float32(vs))
    gk16, _ = orc.gather_kv_cache_fp8(kc, vc, table[None, :].astype(np.uint32), cu, orc.BF16,
                                      ks, vs)
    np.testing.assert_array_equal(gk16, orc.f32_to_bf16_bits(gk))


@pytest.mark.parametrize("scales", [(1.0, 1.0), (0.37, 3.1)])
def test_fp8_attention_equals_attention_over_dequantised_cache(scales):
    """Decode and prefill over an fp8 cache equal the same attention over a
    bf16 cache holding bf16(byte * scale), the dequantisation the reference's
    kernels apply (with scale 1 every E4M3 value is exact in bf16)."""
    ks, vs = scales
    rng = np.random.default_rng(5)
    h, kvh, d, bs, nb = 8, 4, 64, 16, 40
    kc8 = rng.integers(0, 256, size=(nb, kvh, d // 16, bs, 16), dtype=np.uint8)
    vc8 = rng.integers(0, 256, size=(nb, kvh, d, bs), dtype=np.uint8)
    kc8[(kc8 & 0x7F) == 0x7F] = 0x38  # no NaN codes
    vc8[(vc8 & 0x7F) == 0x7F] = 0x38
    kdq = orc.f32_to_bf16_bits(orc.fp8_to_f32(kc8) * np.float32(ks))
    kc16 = np.ascontiguousarray(
        kdq.reshape(nb, kvh, d // 16, bs, 2, 8).transpose(0, 1, 2, 4, 3, 5).reshape(
            nb, kvh, d // 8, bs, 8))
    vc16 = orc.f32_to_bf16_bits(orc.fp8_to_f32(vc8) * np.float32(vs))
    lens = np.array([1, 40, 129, 300], dtype=np.uint32)
    bt = np.stack([rng.permutation(nb)[:19] for _ in lens]).astype(np.uint32)
    q = orc.from_f32(rng.standard_normal((len(lens), h, d)).astype(np.float32), orc.BF16)
    got = orc.paged_attention(q, kc8, vc8, bt, lens, 304, 0.1, dtype=orc.BF16, kv_dtype=orc.FP8,
                              k_scale=ks, v_scale=vs)
    want = orc.paged_attention(q, kc16, vc16, bt, lens, 304, 0.1, dtype=orc.BF16)
    np.testing.assert_array_equal(got, want)
    cu = np.array([0, 1, 5, 20, 27], dtype=np.uint32)
    qp = orc.from_f32(rng.standard_normal((27, h, d)).astype(np.float32), orc.BF16)
    got = orc.prefill_attention(qp, kc8, vc8, bt, lens, cu, 0.1, dtype=orc.BF16,
                                kv_dtype=orc.FP8, k_scale=ks, v_scale=vs)
    want = orc.prefill_attention(qp, kc16, vc16, bt, lens, cu, 0.1, dtype=orc.BF16)
    np.testing.assert_array_equal(got, want)


# ---- next-token selection and EOS state ---------------------------------------

def test_argmax_oracle_matches_numpy_first_maximum():
    """Without NaN, candle's strictly-greater scan is numpy's argmax (first
    occurrence of the maximum); ties are planted so the first-wins rule is
    exercised."""
    rng = np.random.default_rng(8)
    x = rng.standard_normal((64, 1000)).astype(np.float32)
    for r in range(64):
        m = x[r].max() + 1.0
        x[r, rng.choice(1000, size=1 + r % 4, replace=False)] = m
    np.testing.assert_array_equal(orc.argmax_rows(x), np.argmax(x, axis=1))
    xb = orc.from_f32(x, orc.BF16)  # bf16 rounding creates more ties
    np.testing.assert_array_equal(orc.argmax_rows(xb, dtype=orc.BF16),
                                  np.argmax(orc.to_f32(xb, orc.BF16), axis=1))


def test_argmax_oracle_nan_and_infinity_rule():
    x = np.float32([[np.nan, 5, 1], [0, np.nan, 7], [-np.inf] * 3, [np.nan] * 3, [2, 2, np.inf]])
    np.testing.assert_array_equal(orc.argmax_rows(x), [0, 2, 0, 0, 2])


def test_argmax_oracle_nan_rows_against_nanargmax():
    """Rows with NaN scattered in them (and ties, infinities): the scan's rule
    is numpy's nanargmax (the first maximum of the non-NaN elements), except
    that a NaN in element 0 is kept (nothing compares greater than it)."""
    rng = np.random.default_rng(9)
    x = rng.standard_normal((200, 300)).astype(np.float32)
    for r in range(200):
        x[r, rng.choice(300, size=rng.integers(1, 60), replace=False)] = np.nan
        if r % 5 == 0:
            x[r, rng.choice(300, size=3, replace=False)] = np.inf
        if r % 7 == 0:
            x[r, 0] = np.nan
        if r % 11 == 0:  # ties of the row's maximum
            m = np.nanmax(x[r])
            x[r, rng.choice(300, size=2, replace=False)] = m
    want = np.array([0 if np.isnan(row[0]) else np.nanargmax(row) for row in x])
    np.testing.assert_array_equal(orc.argmax_rows(x), want)
    xb = orc.from_f32(x, orc.BF16)
    xf = orc.to_f32(xb, orc.BF16)
    want_b = np.array([0 if np.isnan(row[0]) else np.nanargmax(row) for row in xf])
    np.testing.assert_array_equal(orc.argmax_rows(xb, dtype=orc.BF16), want_b)


def _reference_decode_loop(pending, steps_logits_ids, eos_ids):
    """The reference's host loop (paged_batch_engine.rs:640-667 and :722):
    active rows are compacted; a pending EOS id finishes its row, others are
    pushed to `generated` and fed; the forward's argmax of the fed rows
    becomes their pending id."""
    batch = len(pending)
    next_ids = list(pending)
    finished = [False] * batch
    generated = [[] for _ in range(batch)]
    for new_ids in steps_logits_ids:
        forward = [i for i in range(batch) if not finished[i]]
        fed = []
        for i in forward:
            tok = next_ids[i]
            if tok in eos_ids:
                finished[i] = True
                continue
            generated[i].append(tok)
            fed.append(i)
        for i in fed:
            next_ids[i] = int(new_ids[i])
    return finished, generated


def _reference_decode_loop_with_stalls(pending, steps_new_ids, stalls, eos_ids):
    """paged_batch_engine.rs:209-300 with allocation failures: a slot whose
    try_allocate_slots fails at a step is not decodable, stays out of the
    forward and keeps its pending id; decodable slots consume their pending
    id (an EOS id finishes the slot), feed it and take the forward's argmax."""
    batch = len(pending)
    next_ids = list(pending)
    finished = [False] * batch
    generated = [[] for _ in range(batch)]
    for n, new_ids in enumerate(steps_new_ids):
        for i in range(batch):
            if finished[i] or i in stalls[n]:
                continue
            tok = next_ids[i]
            if tok in eos_ids:
                finished[i] = True
                continue
            generated[i].append(tok)
            next_ids[i] = int(new_ids[i])
    return finished, generated


def test_consume_oracle_with_stalls_equals_reference_loop():
    """Rows whose block allocation fails: the device loop consumes before it
    allocates, so a row that then stalls has appended its token already; the
    next step's consume sees the row's PAD slot, feeds the same input again
    and drops the pending id of the forward the row took no part in. The
    generated lists and finished flags end equal to the reference's, where a
    slot that cannot allocate is skipped with its pending id kept."""
    rng = np.random.default_rng(17)
    batch, steps, cap = 29, 16, 24
    eos = [2, 5]
    pending = rng.integers(0, 9, size=batch)
    new_ids = [rng.integers(0, 9, size=batch) for _ in range(steps)]
    stalls = [set(rng.choice(batch, size=int(rng.integers(0, 8)), replace=False).tolist())
              for _ in range(steps - 1)] + [set()]  # the last step serves every row
    want_fin, want_gen = _reference_decode_loop_with_stalls(list(pending), new_ids, stalls, eos)
    nid = pending.astype(np.uint32)
    fin = np.zeros(batch, np.uint8)
    gen = np.zeros((batch, cap), np.uint32)
    glen = np.zeros(batch, np.uint32)
    inp = np.zeros(batch, np.uint32)
    prev = np.zeros(batch, np.int64)  # admission: every row counts as having run
    stalled_rows_seen = 0
    for n in range(steps):
        inp, active = orc.decode_consume_tokens(nid, fin, gen, glen, eos, eos[0], prev, inp)
        assert active == int((fin == 0).sum())
        ran = np.array([not fin[i] and i not in stalls[n] for i in range(batch)])
        stalled_rows_seen += int((~ran & (fin == 0)).sum())
        prev = np.where(ran, 0, -1).astype(np.int64)
        # forward + argmax over every row; stalled rows get a junk id
        nid = np.where(ran, new_ids[n], 1 << 30).astype(np.uint32)
    assert stalled_rows_seen > 0
    assert fin.astype(bool).tolist() == want_fin
    assert [gen[i, :glen[i]].tolist() for i in range(batch)] == want_gen


def test_consume_oracle_equals_reference_loop_with_compaction():
    """Feeding finished rows the fill id instead of compacting them gives the
    reference's generated lists and finished flags after every step."""
    rng = np.random.default_rng(9)
    batch, steps, cap = 37, 12, 16
    eos = [2, 5]
    pending = rng.integers(0, 8, size=batch)
    new_ids = [rng.integers(0, 8, size=batch) for _ in range(steps)]
    want_fin, want_gen = _reference_decode_loop(list(pending), new_ids, eos)
    nid = pending.astype(np.uint32)
    fin = np.zeros(batch, np.uint8)
    gen = np.zeros((batch, cap), np.uint32)
    glen = np.zeros(batch, np.uint32)
    for s in range(steps):
        inp, active = orc.decode_consume_tokens(nid, fin, gen, glen, eos, eos[0])
        assert active == int((fin == 0).sum())
        assert np.all(inp[fin == 1] == eos[0])
        nid = np.where(fin == 0, new_ids[s], nid).astype(np.uint32)  # forward + argmax
    assert fin.astype(bool).tolist() == want_fin
    assert [gen[i, :glen[i]].tolist() for i in range(batch)] == want_gen


# ---- block manager restatement (paged_cache_runtime.rs:217-371) -------------

def test_oracle_block_manager_reference_kats():
    """The reference's own KATs (paged_cache_runtime.rs:737-778) on the
    oracle's restatement."""
    m = orc.BlockManager(8, 4)                      # :737-752
    assert m.free_blocks() == 7
    m.allocate_slots(10, 5)
    assert len(m.block_ids(10)) == 2 and m.free_blocks() == 5
    m.allocate_slots(10, 9)
    assert len(m.block_ids(10)) == 3 and m.free_blocks() == 4
    m.free_request(10)
    assert m.free_blocks() == 7
    m = orc.BlockManager(8, 4)                      # :755-769
    m.allocate_slots(10, 12)
    assert len(m.block_ids(10)) == 3 and m.free_blocks() == 4
    m.trim_request_to_num_tokens(10, 5)
    assert len(m.block_ids(10)) == 2 and m.free_blocks() == 5
    m.trim_request_to_num_tokens(10, 1)
    assert len(m.block_ids(10)) == 1 and m.free_blocks() == 6
    m = orc.BlockManager(4, 4)                      # :772-778
    assert m.try_allocate_slots(1, 4)
    assert not m.try_allocate_slots(2, 16)
    assert m.free_blocks() == 2
    with pytest.raises(orc.OracleError, match="paged KV cache exhausted"):
        m.allocate_slots(2, 16)
    assert orc.BlockManager.allocatable_block_capacity(8) == 7


def test_oracle_block_manager_free_list_order():
    """FIFO hand-out from the front, freed and trimmed tails returned to the
    back last block first (VecDeque push_back of the reversed tail,
    paged_cache_runtime.rs:322-359); block 0 never handed out."""
    m = orc.BlockManager(8, 4)
    m.allocate_slots(1, 8)
    m.allocate_slots(2, 4)
    assert m.block_ids(1) == [1, 2] and m.block_ids(2) == [3]
    m.free_request(1)
    m.allocate_slots(3, 24)
    assert m.block_ids(3) == [4, 5, 6, 7, 2, 1]
    m.trim_request_to_num_tokens(3, 9)
    m.allocate_slots(4, 12)
    assert m.block_ids(4) == [1, 2, 7] and m.block_ids(3) == [4, 5, 6]
    assert m.total_allocated_blocks() == 7 and m.free_blocks() == 0
    assert m.slots_available_for(3, 12) and not m.slots_available_for(3, 13)
    assert m.try_allocate_slots(5, 0) and m.blocks_for_request(5) == 0
    with pytest.raises(orc.OracleError):
        m.block_ids(99)
    assert orc.slot_for_position([3, 9], 4, 10, 6) == 9 * 4 + 2
    with pytest.raises(orc.OracleError, match="missing block table entry"):
        orc.slot_for_position([3, 9], 4, 10, 8)
    with pytest.raises(orc.OracleError, match="exceeds paged cache capacity"):
        orc.slot_for_position([3, 12], 4, 10, 5)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_host_block_manager_equals_oracle_restatement(seed):
    """The library's host block manager (C ABI, csrc/host_metadata.cpp) and
    the oracle's pure-Python restatement stay equal through a random run of
    grows, trims, frees and exhaustion."""
    from vpa import host
    rng = np.random.default_rng(seed)
    nb, bs = 40, 8
    a, b = host.BlockManager(nb, bs), orc.BlockManager(nb, bs)
    tokens = {}
    for _ in range(400):
        rid = int(rng.integers(0, 12))
        op = rng.random()
        if op < 0.55:
            n = tokens.get(rid, 0) + int(rng.integers(0, 3 * bs))
            ok_a, ok_b = a.try_allocate_slots(rid, n), b.try_allocate_slots(rid, n)
            assert ok_a == ok_b
            if ok_a:
                tokens[rid] = max(tokens.get(rid, 0), n)
        elif op < 0.8:
            n = int(rng.integers(0, tokens.get(rid, 0) + 1))
            a.trim_request_to_num_tokens(rid, n)
            b.trim_request_to_num_tokens(rid, n)
            if rid in tokens:
                tokens[rid] = min(tokens[rid], n)
        else:
            a.free_request(rid)
            b.free_request(rid)
            tokens.pop(rid, None)
        assert a.free_blocks() == b.free_blocks()
        assert a.total_allocated_blocks() == b.total_allocated_blocks()
        for r in range(12):
            assert a.blocks_for_request(r) == b.blocks_for_request(r)
            if b.blocks_for_request(r):
                assert a.block_ids(r) == b.block_ids(r)
